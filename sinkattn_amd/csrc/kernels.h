// Kernel argument blocks and launchers shared between the .hip sources and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sa {

struct PlanArgs {
  const uint8_t* mask;
  int64_t ms[4];
  int H, nqb, nkb, rows;
  int32_t* counts;
  int32_t* idx;
  int32_t* order;
};

struct FwdArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* lse;
  int64_t qs[4], ks[4], vs[4], os[4];
  const int32_t* counts;
  const int32_t* idx;
  const int32_t* order;
  int B, H, Nq, Nk, nqb, nkb;
  float scale;
};

struct PoolArgs {
  const void* q;
  const void* k;
  int64_t qs[4], ks[4];
  int B, H, Hk, Nq, Nk, nqb, nkb;
  float scale;
  int causal;
  void* out;  // fp32 map (exact/mean) or q.dtype map (max)
  float* ws;  // workspace (mean mode)
};

struct MaskArgs {
  const float* scores;
  int H, nq, nk;
  float coverage;
  int keep_diagonal;
  int req_q, req_k;
  int mode;
  int text_blocks;
  uint8_t* mask;
  int32_t* counts;
  int32_t* idx;
  int32_t* ws_top1;   // [H*nq] workspace
  uint8_t* ws_flags;  // [H*nq] workspace
};

constexpr int kXcds = 8;  // gfx950: work-group i is dispatched to XCD i % 8
int plan_order_slots(int rows, int nqb);
hipError_t launch_block_sparse_plan(const PlanArgs& a, hipStream_t stream);
hipError_t launch_block_sparse_fwd(const FwdArgs& a, int dtype, int D, hipStream_t stream);
hipError_t launch_block_mass_pool(const PoolArgs& a, int dtype, int D, hipStream_t stream);
int block_mass_groups();
hipError_t launch_max_pool(const PoolArgs& a, int dtype, int D, hipStream_t stream);
hipError_t launch_mean_pool(const PoolArgs& a, int dtype, int D, hipStream_t stream);
hipError_t launch_coverage_mask(const MaskArgs& a, hipStream_t stream);

}  // namespace sa
