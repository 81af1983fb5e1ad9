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
  // Launch-order cache (nullptr: none): orders of earlier plans of this shape, keyed by a
  // hash of their tile counts; see plan_order_cache_ints().
  int32_t* cache;
  int cache_entries;
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
  // Compensation tiles (16-bit D=128 kernel): q-blocks below comp_qblocks also attend
  // every key of kd/vd [B,H,Nd,D] (row strides equal to k's/v's; kds/vds = batch and head
  // strides) with comp_bias added to the log2-domain logits.  comp_qblocks = 0: none.
  const void* kd;
  const void* vd;
  int64_t kds[2], vds[2];
  int Nd, comp_qblocks;
  float comp_bias;
};

struct PoolArgs {
  const void* q;
  const void* k;
  int64_t qs[4], ks[4];
  int B, H, Hk, Nq, Nk, nqb, nkb;
  int bs, D;  // block size, head dim
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
  uint8_t* ws_flags;  // [H*nq] workspace (empty-row and top-tie flags), padded to 256 B
};

// Token mean pooling: rows [0, prefix) copied, then groups of `gap` rows averaged
// (a short last group repeats row N-1).  x [B,H,N,D] -> out [B,H,Nout,D].
struct TokenPoolArgs {
  const void* x;
  int64_t xs[4];
  void* out;
  int64_t os[4];
  int B, H, N, D, Nout, prefix, gap;
};

// out = a*sink + (1-a)*dyn with a = sigmoid(lse_s - lse_d - log_gap), per-op rounding.
struct MixArgs {
  const void* sink;
  const void* dyn;
  const void* lse_s;
  const void* lse_d;
  void* out;
  int64_t ss[4], ds[4], lss[3], lds[3], os[4];
  int B, H, N, D;
  float log_gap;
};

// RMSNorm (weights w, eps) over rows of C channels, then rotation of the channel pairs
// of every D-channel head by the table row (row / rows_per_pos) % freq_rows.
struct QkPrepArgs {
  const void* q_in;
  const void* k_in;
  void* q_out;
  void* k_out;
  int64_t in_stride, out_stride;  // elements between rows
  const float* wq;
  const float* wk;
  float eps_q, eps_k;
  const float* freq_real;  // [freq_rows, D/2] fp32, or null: no rotation
  const float* freq_imag;
  int64_t rows, rows_per_pos, freq_rows;
  int C, D;
};

constexpr int kXcds = 8;  // gfx950: work-group i is dispatched to XCD i % 8
int plan_order_slots(int rows, int nqb);
int64_t plan_order_cache_ints(int rows, int nqb, int entries);
hipError_t launch_block_sparse_plan(const PlanArgs& a, hipStream_t stream);
hipError_t launch_block_sparse_fwd(const FwdArgs& a, int dtype, int D, hipStream_t stream);
hipError_t launch_block_mass_pool(const PoolArgs& a, int dtype, int D, hipStream_t stream);
int block_mass_groups();
int device_cu_count();
// Resident work-groups of the persistent max-pool kernel: its workspace holds one slot per
// group, so the launch and the workspace query both use this count.
int max_pool_groups();
hipError_t launch_max_pool(const PoolArgs& a, int dtype, int D, hipStream_t stream);
hipError_t launch_mean_pool(const PoolArgs& a, int dtype, int D, hipStream_t stream);
// Any block size / head dim (pooling_generic.hip); LDS need, checked by the caller against
// kGenericPoolMaxLds.
constexpr size_t kGenericPoolMaxLds = 160 * 1024;
size_t generic_pool_lds_need(int D, int nkb, int dtype);
hipError_t launch_block_mass_generic(const PoolArgs& a, int dtype, hipStream_t stream);
hipError_t launch_max_pool_generic(const PoolArgs& a, int dtype, hipStream_t stream);
hipError_t launch_coverage_mask(const MaskArgs& a, hipStream_t stream);
hipError_t launch_mean_pool_tokens(const TokenPoolArgs& a, int dtype, hipStream_t stream);
hipError_t launch_lse_mix(const MixArgs& a, int dtype, hipStream_t stream);
hipError_t launch_qk_prep(const QkPrepArgs& a, int dtype, hipStream_t stream);

// The C ABI's status channel (capi.cpp): api_fail stores a printf-style message for
// sinkattn_last_error() and returns -1; api_hip_status returns 0 for hipSuccess, else stores
// "<what>: <HIP message>" and returns the error code.
int api_fail(const char* fmt, ...);
int api_hip_status(hipError_t e, const char* what);

}  // namespace sa
