// QK-norm + rotary embedding in front of the sparse attention, gfx950.
//
// The reference runs them as two Triton kernels (wanx/runtime/fast_misc.py:308-340 RMSNorm,
// 432-500 rotary) or as torch ops, each a full read and write of Q and K.  Here one pass:
//   rstd = 1 / sqrt(sum(x^2) / C + eps)            fp32
//   y    = dtype(x * rstd * w)                     (the norm's output tensor)
//   out  = dtype(rotate(y, real, imag))            pairs (2i, 2i+1) of every head:
//          (y0*re - y1*im, y0*im + y1*re)
// Q and K rows are read once and written once (16 bytes per lane per access).  A row is
// handled by a group of GS lanes (GS = 64 for rows of more than 64 chunks of 16 bytes,
// else the next power of two >= the chunk count, so a wave takes 64 / GS rows at once).
// Each wave walks rows with a stride of the whole grid and keeps its lanes' norm weights
// in registers for the whole walk; the rotation table row [D/2] (fp32 real, imag) is
// shared by the heads of a position.

#include "common.h"
#include "kernels.h"

namespace sa {

// SHARED: GS is a multiple of a head's chunk count, so all chunks of a lane sit at the
// same offset within their heads and need the same table entries (loaded once per row).
template <int IT, int CPL, int GS, bool SHARED>
__global__ __launch_bounds__(256) void qk_prep_kernel(QkPrepArgs a, int64_t row_step) {
  constexpr int ES = ElemSize<IT>::value;
  constexpr int EPC = 16 / ES;  // elements per 16-byte chunk (8 for 16-bit types)
  constexpr int RPW = 64 / GS;  // rows per wave and step
  constexpr int NP = EPC / 8 + (EPC < 8);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int gl = lane % GS, sub = lane / GS;
  const bool is_q = blockIdx.y == 0;
  const char* in = (const char*)(is_q ? a.q_in : a.k_in);
  char* out = (char*)(is_q ? a.q_out : a.k_out);
  const float* w = is_q ? a.wq : a.wk;
  const float eps = is_q ? a.eps_q : a.eps_k;
  const int chunks = a.C / EPC;
  const bool rot = a.freq_real != nullptr;

  // this lane's norm weights, loaded once
  f32x4 wv[CPL][EPC / 4];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = gl + GS * i;
#pragma unroll
    for (int j = 0; j < EPC / 4; ++j)
      wv[i][j] = c < chunks ? *reinterpret_cast<const f32x4*>(w + c * EPC + 4 * j) : f32x4{};
  }

  // Wave-uniform walk: every lane takes part in the reductions; rows past the end only
  // skip their loads and stores.
  for (int64_t base = ((int64_t)blockIdx.x * 4 + wave) * RPW; base < a.rows; base += row_step) {
    const int64_t row = base + sub;
    const bool live = row < a.rows;
    const char* src = in + row * a.in_stride * ES;
    char* dst = out + row * a.out_stride * ES;
    // position of this row in the rotation table
    const int64_t frow = rot ? (row / a.rows_per_pos) % a.freq_rows : 0;
    const float* fre = a.freq_real + frow * (a.D / 2);
    const float* fim = a.freq_imag + frow * (a.D / 2);
    // every load of the row up front (x and table entries, 16 bytes each), so their
    // latencies overlap; the reduction then runs on registers
    u32x4 xv[CPL];
    f32x4 rv[CPL][NP], iv[CPL][NP];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = gl + GS * i;
      xv[i] = u32x4{0, 0, 0, 0};
      if (live && c < chunks) {
        const int col = c * EPC;
        xv[i] = *reinterpret_cast<const u32x4*>(src + c * 16);
        if (rot && (i == 0 || !SHARED)) {
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
#pragma unroll
    for (int m = GS / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
    const float rstd = 1.0f / sqrtf(ss / (float)a.C + eps);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = gl + GS * i;
      if (live && c < chunks) {
        float o[EPC];
#pragma unroll
        for (int pr = 0; pr < EPC / 2; ++pr) {
          // the norm's output is a tensor of the input dtype: round before rotating
          float y0 = x[i][2 * pr] * rstd * wv[i][(2 * pr) / 4][(2 * pr) % 4];
          float y1 = x[i][2 * pr + 1] * rstd * wv[i][(2 * pr + 1) / 4][(2 * pr + 1) % 4];
          if constexpr (IT == kBF16) { y0 = (float)(__bf16)y0; y1 = (float)(__bf16)y1; }
          if constexpr (IT == kF16) { y0 = (float)(_Float16)y0; y1 = (float)(_Float16)y1; }
          if (rot) {
            const int ti = SHARED ? 0 : i;
            const float re = rv[ti][0][pr], im = iv[ti][0][pr];
            o[2 * pr] = y0 * re - y1 * im;
            o[2 * pr + 1] = y0 * im + y1 * re;
          } else {
            o[2 * pr] = y0;
            o[2 * pr + 1] = y1;
          }
        }
        u32x4 ov;
        if constexpr (IT == kF32) {
#pragma unroll
          for (int j = 0; j < 4; ++j) ov[j] = __float_as_uint(o[j]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) ov[j] = pack2<IT>(o[2 * j], o[2 * j + 1]);
        }
        *reinterpret_cast<u32x4*>(dst + c * 16) = ov;
      }
    }
  }
}

// Position-major walk, for rows of one 16-byte chunk per lane (CPL 1) that share the table
// row of their position: rows_per_pos consecutive rows (the heads of a token) use the same
// rotation entries, so a wave takes one position at a time, loads its lane's entries once,
// and then normalises and rotates that position's rows, 64 / GS of them per step.
template <int IT, int GS>
__global__ __launch_bounds__(256) void qk_prep_pos_kernel(QkPrepArgs a, int64_t npos, int64_t pos_step) {
  constexpr int ES = ElemSize<IT>::value;
  constexpr int EPC = 16 / ES;
  constexpr int RPW = 64 / GS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int gl = lane % GS, sub = lane / GS;
  const bool is_q = blockIdx.y == 0;
  const char* in = (const char*)(is_q ? a.q_in : a.k_in);
  char* out = (char*)(is_q ? a.q_out : a.k_out);
  const float* w = is_q ? a.wq : a.wk;
  const float eps = is_q ? a.eps_q : a.eps_k;
  const int chunks = a.C / EPC;
  const bool has = gl < chunks;
  const int R = (int)a.rows_per_pos;
  f32x4 wv[EPC / 4];
#pragma unroll
  for (int j = 0; j < EPC / 4; ++j)
    wv[j] = has ? *reinterpret_cast<const f32x4*>(w + gl * EPC + 4 * j) : f32x4{};
  const int p0 = ((gl * EPC) % a.D) / 2;  // first pair of this lane's chunk within its head

  for (int64_t pos = (int64_t)blockIdx.x * 4 + wave; pos < npos; pos += pos_step) {
    const int64_t frow = pos % a.freq_rows;
    f32x4 rv = f32x4{}, iv = f32x4{};
    if (has) {
      if constexpr (EPC == 8) {
        rv = *reinterpret_cast<const f32x4*>(a.freq_real + frow * (a.D / 2) + p0);
        iv = *reinterpret_cast<const f32x4*>(a.freq_imag + frow * (a.D / 2) + p0);
      } else {
        const f32x2 r2 = *reinterpret_cast<const f32x2*>(a.freq_real + frow * (a.D / 2) + p0);
        const f32x2 i2 = *reinterpret_cast<const f32x2*>(a.freq_imag + frow * (a.D / 2) + p0);
        rv = f32x4{r2[0], r2[1], 0.f, 0.f};
        iv = f32x4{i2[0], i2[1], 0.f, 0.f};
      }
    }
    for (int h0 = 0; h0 < R; h0 += RPW) {
      const int hh = h0 + sub;
      const bool live = has && hh < R;
      const int64_t row = pos * R + hh;
      u32x4 xv = u32x4{0, 0, 0, 0};
      if (live) xv = *reinterpret_cast<const u32x4*>(in + (row * a.in_stride) * ES + gl * 16);
      float x[EPC];
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (IT == kF32) {
          x[j] = __uint_as_float(xv[j]);
        } else {
          const uint32_t lo = xv[j] & 0xffffu, hi = xv[j] >> 16;
          x[2 * j] = IT == kBF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
          x[2 * j + 1] = IT == kBF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
        }
      }
#pragma unroll
      for (int e = 0; e < EPC; ++e) ss += x[e] * x[e];
#pragma unroll
      for (int m = GS / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
      const float rstd = 1.0f / sqrtf(ss / (float)a.C + eps);
      if (live) {
        float o[EPC];
#pragma unroll
        for (int pr = 0; pr < EPC / 2; ++pr) {
          // the norm's output is a tensor of the input dtype: round before rotating
          float y0 = x[2 * pr] * rstd * wv[(2 * pr) / 4][(2 * pr) % 4];
          float y1 = x[2 * pr + 1] * rstd * wv[(2 * pr + 1) / 4][(2 * pr + 1) % 4];
          if constexpr (IT == kBF16) { y0 = (float)(__bf16)y0; y1 = (float)(__bf16)y1; }
          if constexpr (IT == kF16) { y0 = (float)(_Float16)y0; y1 = (float)(_Float16)y1; }
          o[2 * pr] = y0 * rv[pr] - y1 * iv[pr];
          o[2 * pr + 1] = y0 * iv[pr] + y1 * rv[pr];
        }
        u32x4 ov;
        if constexpr (IT == kF32) {
#pragma unroll
          for (int j = 0; j < 4; ++j) ov[j] = __float_as_uint(o[j]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) ov[j] = pack2<IT>(o[2 * j], o[2 * j + 1]);
        }
        *reinterpret_cast<u32x4*>(out + (row * a.out_stride) * ES + gl * 16) = ov;
      }
    }
  }
}

// grid.y = 0 for Q, 1 for K; grid.x work-groups of four waves, at most eight per CU.
template <int IT, int CPL, int GS>
static hipError_t launch_qk_prep_g(const QkPrepArgs& a, hipStream_t stream) {
  constexpr int EPC = IT == kF32 ? 4 : 8;
  constexpr int RPW = 64 / GS;
  const int64_t need = (a.rows + 4 * RPW - 1) / (4 * RPW);
  const int64_t cap = (int64_t)8 * device_cu_count();
  const int gx = (int)(need < cap ? need : cap);
  const dim3 grid((unsigned)gx, 2);
  const int64_t step = (int64_t)gx * 4 * RPW;
  if (GS % (a.D / EPC) == 0)
    qk_prep_kernel<IT, CPL, GS, true><<<grid, 256, 0, stream>>>(a, step);
  else
    qk_prep_kernel<IT, CPL, GS, false><<<grid, 256, 0, stream>>>(a, step);
  return hipGetLastError();
}

// The position-major kernel: rotation on, one chunk per lane, the lanes of a row on whole
// heads (their table entries repeat per head), and positions of at least two steps of rows.
template <int IT, int GS>
static bool launch_qk_prep_pos(const QkPrepArgs& a, hipStream_t stream, hipError_t* err) {
  constexpr int EPC = IT == kF32 ? 4 : 8;
  constexpr int RPW = 64 / GS;
  const int64_t R = a.rows_per_pos;
  if (a.freq_real == nullptr || R < 2 * RPW || a.rows % R != 0 || GS % (a.D / EPC) != 0) return false;
  const int64_t npos = a.rows / R;
  const int64_t need = (npos + 3) / 4;
  const int64_t cap = (int64_t)8 * device_cu_count();
  const int gx = (int)(need < cap ? need : cap);
  qk_prep_pos_kernel<IT, GS><<<dim3((unsigned)gx, 2), 256, 0, stream>>>(a, npos, (int64_t)gx * 4);
  *err = hipGetLastError();
  return true;
}

template <int IT>
static hipError_t launch_qk_prep_t(const QkPrepArgs& a, hipStream_t stream) {
  constexpr int EPC = IT == kF32 ? 4 : 8;
  const int chunks = a.C / EPC;
  hipError_t err = hipSuccess;
  if (chunks <= 8 && launch_qk_prep_pos<IT, 8>(a, stream, &err)) return err;
  if (chunks > 8 && chunks <= 16 && launch_qk_prep_pos<IT, 16>(a, stream, &err)) return err;
  if (chunks > 16 && chunks <= 32 && launch_qk_prep_pos<IT, 32>(a, stream, &err)) return err;
  if (chunks <= 8) return launch_qk_prep_g<IT, 1, 8>(a, stream);
  if (chunks <= 16) return launch_qk_prep_g<IT, 1, 16>(a, stream);
  if (chunks <= 32) return launch_qk_prep_g<IT, 1, 32>(a, stream);
  if (chunks <= 64) return launch_qk_prep_g<IT, 1, 64>(a, stream);
  if (chunks <= 128) return launch_qk_prep_g<IT, 2, 64>(a, stream);
  if (chunks <= 192) return launch_qk_prep_g<IT, 3, 64>(a, stream);
  if (chunks <= 256) return launch_qk_prep_g<IT, 4, 64>(a, stream);
  if (chunks <= 512) return launch_qk_prep_g<IT, 8, 64>(a, stream);
  return launch_qk_prep_g<IT, 16, 64>(a, stream);
}

hipError_t launch_qk_prep(const QkPrepArgs& a, int dtype, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  if (dtype == kBF16) return launch_qk_prep_t<kBF16>(a, stream);
  if (dtype == kF16) return launch_qk_prep_t<kF16>(a, stream);
  return launch_qk_prep_t<kF32>(a, stream);
}

}  // namespace sa
