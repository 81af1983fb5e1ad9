// Measurement probe for bench.py (built into libsinkattn_probe.so, not into libsinkattn).
//
// The exact block-mass pooling kernel (block_mass_persistent_kernel) spends, per score, one
// v_fma_f32 (scale and reference maximum), one v_exp_f32 and one v_add_f32 (the block sum),
// besides the MFMA that produced the score.  This kernel issues exactly that mix from
// registers, 16 independent chains per lane, with the pooling kernel's occupancy (three
// 256-thread groups per CU), so that bench.py can measure the rate at which a CU retires the
// mix (scores per shader clock per CU) and price the pooling pass's algorithmic VALU work
// (B*H*Nq*Nk scores) against it.  Each wave also stamps s_memtime (shader clock) and
// s_memrealtime (100 MHz) around its loop, which gives the clock the mix ran at.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kChains = 16;

// 48 KB of LDS per group: at most three groups fit a CU's 160 KB, as for the pooling
// kernel, so a launch of three groups per CU puts exactly three on every CU.
constexpr int kPadFloats = 12288;

__global__ __launch_bounds__(256, 3) void valu_mix_kernel(int reps, float c, float* sink, long long* stamps) {
  __shared__ float pad[kPadFloats];
  const int lane = (int)(threadIdx.x & 63);
  pad[threadIdx.x * 48] = (float)lane;
  float s[kChains], acc[kChains];
#pragma unroll
  for (int i = 0; i < kChains; ++i) {
    s[i] = (float)lane * 0.03125f + (float)i * 0.25f - 2.0f;
    acc[i] = 0.f;
  }
  float nm = -1.0f;
  const long long m0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < reps; ++it) {
#pragma unroll
    for (int i = 0; i < kChains; ++i) acc[i] += __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], c, nm));
    nm -= 1.0e-7f;
  }
  const long long m1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float total = pad[threadIdx.x * 48];
#pragma unroll
  for (int i = 0; i < kChains; ++i) total += acc[i];
  sink[blockIdx.x * blockDim.x + threadIdx.x] = total;
  if (lane == 0) {
    long long* st = stamps + 3 * (blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6));
    st[0] = m1 - m0;
    st[1] = r0;
    st[2] = r1;
  }
}

}  // namespace

extern "C" {

// Scores one launch issues: blocks * 256 * reps * 16.  sink: blocks * 256 floats; stamps:
// blocks * 4 * 3 int64 (per wave: shader cycles of its loop, real-time start and end).
int sinkattn_probe_valu_mix(int blocks, int reps, float c, float* sink, long long* stamps, void* stream) {
  if (blocks <= 0 || reps <= 0 || sink == nullptr || stamps == nullptr) return -1;
  valu_mix_kernel<<<blocks, 256, 0, (hipStream_t)stream>>>(reps, c, sink, stamps);
  return (int)hipGetLastError();
}

int sinkattn_probe_chains(void) { return kChains; }

}  // extern "C"
