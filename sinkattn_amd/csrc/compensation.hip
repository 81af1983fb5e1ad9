// Compensation branch of the sink-sparse layer call, gfx950.
//
// The reference runs it as torch ops after the sparse call
// (sinkattention/sparse_attention.py:79-115 pooling, 898-919 mix;
// wanx/runtime/sink_sparse_wan.py:210-265):
//   K', V'  = K, V with rows [prefix, N) mean-pooled in groups of `gap` (a short last
//             group repeats the last row: replicate padding)
//   out_d   = attention(Q, K', V') with LSE
//   out     = a * out_s + (1 - a) * out_d,  a = sigmoid(lse_s - lse_d - ln gap)
//
// This file holds the two HBM-bound pieces:
//   mean_pool_tokens_kernel  K or V -> pooled rows (reads the input once, 16 bytes per
//                            lane per row, fp32 sums, one rounding at the end)
//   lse_mix_kernel           the mix with the reference's rounding: every torch op of the
//                            reference is one fp32 operation rounded to the tensor dtype
// The attention over the pooled keys runs in block_sparse_fwd.hip, either as a separate
// all-blocks call or fused into the sparse call (the "compensation tiles").

#include "common.h"
#include "kernels.h"

// The mix restates torch ops one by one: no fused multiply-adds.
#pragma clang fp contract(off)

namespace sa {

// ---------------------------------------------------------------------------------------
// Token mean pooling.  One 256-lane work-group covers 256 / C output rows of one (b, h),
// C = 16-byte chunks per row; lane (row r, chunk c) sums chunk c of the input rows of r.
// ---------------------------------------------------------------------------------------
template <int IT>
__device__ __forceinline__ void add_chunk(float* acc, const char* p) {
  const u32x4 w = *reinterpret_cast<const u32x4*>(p);
  if constexpr (IT == kF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += __uint_as_float(w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = w[i] & 0xffffu, hi = w[i] >> 16;
      acc[2 * i] += IT == kBF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
      acc[2 * i + 1] += IT == kBF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
    }
  }
}

template <int IT>
__global__ __launch_bounds__(256) void mean_pool_tokens_kernel(TokenPoolArgs a) {
  constexpr int ES = ElemSize<IT>::value;
  constexpr int EPC = 16 / ES;  // elements per 16-byte chunk
  const int chunks = a.D / EPC;
  const int rows_per_wg = 256 / chunks;
  const int c = threadIdx.x % chunks;
  const int r = blockIdx.x * rows_per_wg + threadIdx.x / chunks;
  const int bh = blockIdx.y;
  if (r >= a.Nout) return;
  const int b = bh / a.H, h = bh - b * a.H;
  const char* xb = (const char*)a.x + ((int64_t)b * a.xs[0] + (int64_t)h * a.xs[1]) * ES + c * 16;
  char* ob = (char*)a.out + ((int64_t)b * a.os[0] + (int64_t)h * a.os[1] + (int64_t)r * a.os[2]) * ES + c * 16;
  if (r < a.prefix) {  // kept rows
    *reinterpret_cast<u32x4*>(ob) = *reinterpret_cast<const u32x4*>(xb + (int64_t)r * a.xs[2] * ES);
    return;
  }
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int g0 = a.prefix + (r - a.prefix) * a.gap;
  const int last = a.N - 1;
  for (int j = 0; j < a.gap; ++j) {
    const int row = min(g0 + j, last);
    add_chunk<IT>(acc, xb + (int64_t)row * a.xs[2] * ES);
  }
  // torch's mean: fp32 sum times the fp32 factor 1/gap, one rounding to the dtype
  const float f = 1.0f / (float)a.gap;
  if constexpr (IT == kF32) {
    *reinterpret_cast<f32x4*>(ob) = f32x4{acc[0] * f, acc[1] * f, acc[2] * f, acc[3] * f};
  } else {
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pack2<IT>(acc[2 * i] * f, acc[2 * i + 1] * f);
    *reinterpret_cast<u32x4*>(ob) = o;
  }
}

hipError_t launch_mean_pool_tokens(const TokenPoolArgs& a, int dtype, hipStream_t stream) {
  const int es = dtype == kF32 ? 4 : 2;
  const int chunks = a.D * es / 16;
  const int rows_per_wg = 256 / chunks;
  dim3 grid((a.Nout + rows_per_wg - 1) / rows_per_wg, a.B * a.H);
  if (dtype == kBF16) mean_pool_tokens_kernel<kBF16><<<grid, 256, 0, stream>>>(a);
  else if (dtype == kF16) mean_pool_tokens_kernel<kF16><<<grid, 256, 0, stream>>>(a);
  else mean_pool_tokens_kernel<kF32><<<grid, 256, 0, stream>>>(a);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// LSE mix with the reference's per-op rounding.  For 16-bit dtypes every step below is
// one torch op on a bf16/f16 tensor there: computed in fp32 and rounded to the dtype.
//   lg   = round(log(round(gap)))                   sink_lse.new_tensor(gap).log()
//   wd   = round(lse_d + lg);  mx = max(lse_s, wd)
//   es   = round(exp(round(lse_s - mx)));  ed = round(exp(round(wd - mx)))
//   a    = round(es / round(es + ed));  na = round(1 - a)
//   out  = round(round(o_s * a) + round(o_d * na))
// One lane per 8 channels; a wave covers 512 channels of one row or several rows.
// ---------------------------------------------------------------------------------------
template <int IT>
__device__ __forceinline__ float rnd(float x) {
  if constexpr (IT == kBF16) return (float)(__bf16)x;
  else if constexpr (IT == kF16) return (float)(_Float16)x;
  else return x;
}

template <int IT>
__device__ __forceinline__ float load_elem(const char* p) {
  if constexpr (IT == kBF16) return bf16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p));
  else if constexpr (IT == kF16) return f16_bits_to_f32(*reinterpret_cast<const uint16_t*>(p));
  else return *reinterpret_cast<const float*>(p);
}

template <int IT>
__global__ __launch_bounds__(256) void lse_mix_kernel(MixArgs a) {
  constexpr int ES = ElemSize<IT>::value;
  constexpr int EPC = 16 / ES;
  const int chunks = a.D / EPC;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / chunks;
  const int c = (int)(gid - row * chunks);
  if (row >= (int64_t)a.B * a.H * a.N) return;
  const int n = (int)(row % a.N);
  const int bh = (int)(row / a.N);
  const int b = bh / a.H, h = bh - b * a.H;
  const float ls = load_elem<IT>((const char*)a.lse_s + ((int64_t)b * a.lss[0] + (int64_t)h * a.lss[1] + (int64_t)n * a.lss[2]) * ES);
  const float ld = load_elem<IT>((const char*)a.lse_d + ((int64_t)b * a.lds[0] + (int64_t)h * a.lds[1] + (int64_t)n * a.lds[2]) * ES);
  const float wd = rnd<IT>(ld + a.log_gap);
  const float mx = fmaxf(ls, wd);
  const float es = rnd<IT>(expf(rnd<IT>(ls - mx)));
  const float ed = rnd<IT>(expf(rnd<IT>(wd - mx)));
  const float al = rnd<IT>(es / rnd<IT>(es + ed));
  const float na = rnd<IT>(1.0f - al);
  const char* ps = (const char*)a.sink + ((int64_t)b * a.ss[0] + (int64_t)h * a.ss[1] + (int64_t)n * a.ss[2]) * ES + c * 16;
  const char* pd = (const char*)a.dyn + ((int64_t)b * a.ds[0] + (int64_t)h * a.ds[1] + (int64_t)n * a.ds[2]) * ES + c * 16;
  char* po = (char*)a.out + ((int64_t)b * a.os[0] + (int64_t)h * a.os[1] + (int64_t)n * a.os[2]) * ES + c * 16;
  const u32x4 vs = *reinterpret_cast<const u32x4*>(ps);
  const u32x4 vd = *reinterpret_cast<const u32x4*>(pd);
  u32x4 vo;
  if constexpr (IT == kF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vo[i] = __float_as_uint(__uint_as_float(vs[i]) * al + __uint_as_float(vd[i]) * na);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float r2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t bs = (vs[i] >> (16 * e)) & 0xffffu, bd = (vd[i] >> (16 * e)) & 0xffffu;
        const float xs = IT == kBF16 ? bf16_bits_to_f32(bs) : f16_bits_to_f32(bs);
        const float xd = IT == kBF16 ? bf16_bits_to_f32(bd) : f16_bits_to_f32(bd);
        r2[e] = rnd<IT>(xs * al) + rnd<IT>(xd * na);
      }
      vo[i] = pack2<IT>(r2[0], r2[1]);
    }
  }
  *reinterpret_cast<u32x4*>(po) = vo;
}

hipError_t launch_lse_mix(const MixArgs& a, int dtype, hipStream_t stream) {
  const int es = dtype == kF32 ? 4 : 2;
  const int64_t lanes = (int64_t)a.B * a.H * a.N * (a.D * es / 16);
  const int64_t blocks = (lanes + 255) / 256;
  if (dtype == kBF16) lse_mix_kernel<kBF16><<<blocks, 256, 0, stream>>>(a);
  else if (dtype == kF16) lse_mix_kernel<kF16><<<blocks, 256, 0, stream>>>(a);
  else lse_mix_kernel<kF32><<<blocks, 256, 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace sa
