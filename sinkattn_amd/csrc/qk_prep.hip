// QK-norm + rotary embedding in front of the sparse attention, gfx950.
//
// The reference runs them as two Triton kernels (wanx/runtime/fast_misc.py:308-340 RMSNorm,
// 432-500 rotary) or as torch ops, each a full read and write of Q and K.  Here one
// wave per row (a token's C channels for Wan, one head's D channels for Z-Image):
//   rstd = 1 / sqrt(sum(x^2) / C + eps)            fp32
//   y    = dtype(x * rstd * w)                     (the norm's output tensor)
//   out  = dtype(rotate(y, real, imag))            pairs (2i, 2i+1) of every head:
//          (y0*re - y1*im, y0*im + y1*re)
// Q and K rows are read once and written once (16 bytes per lane per access); the
// rotation table row [D/2] (fp32 real, imag) is shared by the heads of a position.

#include "common.h"
#include "kernels.h"

namespace sa {

template <int IT, int CPL>
__device__ __forceinline__ void qk_prep_row(const QkPrepArgs& a, const char* xin, char* xout,
                                            const float* w, float eps, int64_t row, int lane) {
  constexpr int ES = ElemSize<IT>::value;
  constexpr int EPC = 16 / ES;  // elements per 16-byte chunk (8 for 16-bit types)
  const int chunks = a.C / EPC;
  const char* src = xin + row * a.in_stride * ES;
  char* dst = xout + row * a.out_stride * ES;
  const bool rot = a.freq_real != nullptr;
  // position of this row in the rotation table
  const int64_t frow = rot ? (row / a.rows_per_pos) % a.freq_rows : 0;
  const float* fre = a.freq_real + frow * (a.D / 2);
  const float* fim = a.freq_imag + frow * (a.D / 2);
  // every load of the row up front (x, weights, table entries: 16 bytes each), so their
  // latencies overlap; the reduction then runs on registers
  u32x4 xv[CPL];
  f32x4 wv[CPL][EPC / 4];
  f32x4 rv[CPL][EPC / 8 + (EPC < 8)], iv[CPL][EPC / 8 + (EPC < 8)];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) {
      const int col = c * EPC;
      xv[i] = *reinterpret_cast<const u32x4*>(src + c * 16);
#pragma unroll
      for (int j = 0; j < EPC / 4; ++j) wv[i][j] = *reinterpret_cast<const f32x4*>(w + col + 4 * j);
      if (rot) {
        const int p0 = (col % a.D) / 2;  // first pair of this chunk within its head
        if constexpr (EPC == 8) {
          rv[i][0] = *reinterpret_cast<const f32x4*>(fre + p0);
          iv[i][0] = *reinterpret_cast<const f32x4*>(fim + p0);
        } else {  // 2 pairs per fp32 chunk
          const f32x2 r2 = *reinterpret_cast<const f32x2*>(fre + p0);
          const f32x2 i2 = *reinterpret_cast<const f32x2*>(fim + p0);
          rv[i][0] = f32x4{r2[0], r2[1], 0.f, 0.f};
          iv[i][0] = f32x4{i2[0], i2[1], 0.f, 0.f};
        }
      }
    }
  }
  float x[CPL][EPC];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (IT == kF32) {
          x[i][j] = __uint_as_float(xv[i][j]);
        } else {
          const uint32_t lo = xv[i][j] & 0xffffu, hi = xv[i][j] >> 16;
          x[i][2 * j] = IT == kBF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
          x[i][2 * j + 1] = IT == kBF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
        }
      }
#pragma unroll
      for (int e = 0; e < EPC; ++e) ss += x[i][e] * x[i][e];
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
  const float rstd = 1.0f / sqrtf(ss / (float)a.C + eps);
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    if (c < chunks) {
      float o[EPC];
#pragma unroll
      for (int pr = 0; pr < EPC / 2; ++pr) {
        // the norm's output is a tensor of the input dtype: round before rotating
        float y0 = x[i][2 * pr] * rstd * wv[i][(2 * pr) / 4][(2 * pr) % 4];
        float y1 = x[i][2 * pr + 1] * rstd * wv[i][(2 * pr + 1) / 4][(2 * pr + 1) % 4];
        if constexpr (IT == kBF16) { y0 = (float)(__bf16)y0; y1 = (float)(__bf16)y1; }
        if constexpr (IT == kF16) { y0 = (float)(_Float16)y0; y1 = (float)(_Float16)y1; }
        if (rot) {
          const float re = rv[i][0][pr], im = iv[i][0][pr];
          o[2 * pr] = y0 * re - y1 * im;
          o[2 * pr + 1] = y0 * im + y1 * re;
        } else {
          o[2 * pr] = y0;
          o[2 * pr + 1] = y1;
        }
      }
      u32x4 out;
      if constexpr (IT == kF32) {
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = __float_as_uint(o[j]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = pack2<IT>(o[2 * j], o[2 * j + 1]);
      }
      *reinterpret_cast<u32x4*>(dst + c * 16) = out;
    }
  }
}

// grid.x covers rows, four waves (rows) per work-group; grid.y = 0 for Q, 1 for K.
template <int IT, int CPL>
__global__ __launch_bounds__(256) void qk_prep_kernel(QkPrepArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  if (blockIdx.y == 0)
    qk_prep_row<IT, CPL>(a, (const char*)a.q_in, (char*)a.q_out, a.wq, a.eps_q, row, lane);
  else
    qk_prep_row<IT, CPL>(a, (const char*)a.k_in, (char*)a.k_out, a.wk, a.eps_k, row, lane);
}

template <int IT>
static hipError_t launch_qk_prep_t(const QkPrepArgs& a, hipStream_t stream) {
  constexpr int EPC = IT == kF32 ? 4 : 8;
  const int chunks = a.C / EPC;
  const dim3 grid((unsigned)((a.rows + 3) / 4), 2);
  if (chunks <= 64) qk_prep_kernel<IT, 1><<<grid, 256, 0, stream>>>(a);
  else if (chunks <= 128) qk_prep_kernel<IT, 2><<<grid, 256, 0, stream>>>(a);
  else if (chunks <= 256) qk_prep_kernel<IT, 4><<<grid, 256, 0, stream>>>(a);
  else if (chunks <= 512) qk_prep_kernel<IT, 8><<<grid, 256, 0, stream>>>(a);
  else qk_prep_kernel<IT, 16><<<grid, 256, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_qk_prep(const QkPrepArgs& a, int dtype, hipStream_t stream) {
  if (dtype == kBF16) return launch_qk_prep_t<kBF16>(a, stream);
  if (dtype == kF16) return launch_qk_prep_t<kF16>(a, stream);
  return launch_qk_prep_t<kF32>(a, stream);
}

}  // namespace sa
