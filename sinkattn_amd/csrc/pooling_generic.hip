// Block-score kernels for any block size and head dim (the MFMA kernels in pooling.hip
// cover block 128 / head dim 128, the shapes the calibration runs at).
//
// block_mass_generic: `_compute_exact_block_mass_scores` (sinkattention/sparse_attention.py
//   :145-227) for block sizes 1..1024, head dims 1..256, bf16/f16/f32.
// max_pool_generic: `attn_with_pooling` (sinkattention/pooling_kernel.py:11-248) for block
//   sizes 16/32/64/128 and head dims 16..256 (the reference's asserts,
//   pooling_kernel.py:198-207), bf16/f16/f32, GQA, causal.
//
// One 256-thread work-group per (b, h, query block).  Its rows go in groups of 64; for
// each group the keys stream through LDS in tiles of 64 and the 64x64 score tile is formed
// on the matrix cores (16-bit inputs with a head dim that is a multiple of 16: products
// exact, sums fp32) or else as fp32 dot products on the VALU (every thread a 4x4 piece,
// four head-dim elements per 16-byte LDS read).  Four threads per row then walk that row of
// the tile in key order, 16 keys each, so a key block may start and end anywhere in a
// tile.  Two passes over the keys: the first finds each row's maximum (and, for the exact
// mode, its softmax denominator), the second adds the per-block values into an LDS row of
// the query block's map.

#include "common.h"
#include "kernels.h"

namespace sa {

constexpr int kGenRows = 64;  // rows per group
constexpr int kGenKeys = 64;  // keys per tile

template <int IT>
__device__ __forceinline__ float load_elem(const void* base, int64_t off) {
  if constexpr (IT == kF32) return reinterpret_cast<const float*>(base)[off];
  else if constexpr (IT == kBF16) return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[off]);
  else return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[off]);
}

template <int IT>
__device__ __forceinline__ float round_elem(float x) {
  if constexpr (IT == kBF16) return (float)(__bf16)x;
  else if constexpr (IT == kF16) return (float)(_Float16)x;
  else return x;
}

// Row length in LDS.  fp32 rows (VALU scores): the head dim padded to a multiple of 4
// (zeros) plus 4 floats, so rows stay 16-byte aligned and the 16 key rows a wave reads fall
// on distinct banks.  16-bit rows (matrix-core scores, head dim a multiple of 16): the head
// dim plus 8 elements.
__host__ __device__ inline int generic_row_len(int D) { return ((D + 3) & ~3) + 4; }
__host__ __device__ inline int generic_row_len16(int D) { return D + 8; }

// LDS layout: Q rows [64][row], K tile [64][row], score tile fp32 [64][65], map row fp32
// [nkb].  mf: 16-bit rows for the matrix cores.
__host__ __device__ inline size_t generic_pool_lds_bytes(int D, int nkb, bool mf) {
  const size_t rows = mf ? (size_t)(kGenRows + kGenKeys) * generic_row_len16(D) * 2
                         : (size_t)(kGenRows + kGenKeys) * generic_row_len(D) * 4;
  return rows + ((size_t)kGenRows * (kGenKeys + 1) + nkb) * 4;
}

// Stage `n` rows starting at row0 of one head (row stride st elements) as fp32 into dst
// ([rows][LD]); head-dim padding and rows past n are zero.
template <int IT>
__device__ __forceinline__ void stage_rows(float* dst, const void* base, int64_t st, int row0,
                                           int n, int rows, int D, int LD) {
  const int Dp = LD - 4;
  const int step_r = 256 / Dp, step_d = 256 - step_r * Dp;
  int r = (int)threadIdx.x / Dp, d = (int)threadIdx.x - r * Dp;
#pragma unroll 4
  while (r < rows) {
    const float v = (r < n && d < D) ? load_elem<IT>(base, (int64_t)(row0 + r) * st + d) : 0.f;
    dst[r * LD + d] = v;
    d += step_d;
    r += step_r;
    if (d >= Dp) {
      d -= Dp;
      ++r;
    }
  }
}

// 64x64 tile of raw dot products q_r . k_j into St ([64][65]).
__device__ __forceinline__ void score_tile(const float* Qs, const float* Ks, float* St, int LD) {
  const int rq = threadIdx.x >> 4, kq = threadIdx.x & 15;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  const int Dp = LD - 4;
#pragma unroll 2
  for (int d = 0; d < Dp; d += 4) {
    f32x4 qv[4], kv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[i] = *reinterpret_cast<const f32x4*>(Qs + (rq + 16 * i) * LD + d);
#pragma unroll
    for (int j = 0; j < 4; ++j) kv[j] = *reinterpret_cast<const f32x4*>(Ks + (kq + 16 * j) * LD + d);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][j] = __builtin_fmaf(qv[i][e], kv[j][e], acc[i][j]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) St[(rq + 16 * i) * (kGenKeys + 1) + kq + 16 * j] = acc[i][j];
}

// 16-bit rows, 16 bytes per copy (rows of q/k start 16-byte aligned: the C ABI requires
// 16-byte bases and strides that are multiples of 8 elements).
__device__ __forceinline__ void stage_rows16(uint16_t* dst, const void* base, int64_t st, int row0,
                                             int n, int rows, int D) {
  const int cpr = D / 8, LDh = generic_row_len16(D);
  for (int e = threadIdx.x; e < rows * cpr; e += blockDim.x) {
    const int r = e / cpr, c = e - r * cpr;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (r < n) v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + (int64_t)(row0 + r) * st + 8 * c);
    *reinterpret_cast<u32x4*>(dst + r * LDh + 8 * c) = v;
  }
}

// 64x64 tile of raw dot products on the matrix cores: wave w forms rows 32(w/2).. against
// keys 32(w%2).. with v_mfma_f32_32x32x16 (A = 32 query rows, B = 32 key rows; products
// exact, sums fp32, as the reference's matmul of the upcast inputs up to summation order).
template <int IT>
__device__ __forceinline__ void score_tile16(const uint16_t* Q16, const uint16_t* K16, float* St, int D) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int r0 = 32 * (w >> 1), c0 = 32 * (w & 1), LDh = generic_row_len16(D);
  const uint16_t* qp = Q16 + (r0 + l32) * LDh + 8 * hl;
  const uint16_t* kp = K16 + (c0 + l32) * LDh + 8 * hl;
  f32x16 acc = f32x16{};
  for (int k = 0; k < D; k += 16)
    acc = mfma32x32x16<IT>(*reinterpret_cast<const u32x4*>(qp + k), *reinterpret_cast<const u32x4*>(kp + k), acc);
  // register j of lane (hl, l32): row 8(j/4) + 4hl + j%4, key l32
#pragma unroll
  for (int j = 0; j < 16; ++j)
    St[(r0 + 8 * (j >> 2) + 4 * hl + (j & 3)) * (kGenKeys + 1) + c0 + l32] = acc[j];
}

// Q/K staging and the score tile, on the matrix cores (MF) or as fp32 on the VALU.
template <int IT, bool MF>
struct GenTiles {
  void* qv;
  void* kv;
  float* st;
  int D, LD;
  __device__ GenTiles(float* gsm, int D_) : D(D_) {
    if constexpr (MF) {
      LD = generic_row_len16(D);
      uint16_t* q16 = reinterpret_cast<uint16_t*>(gsm);
      qv = q16;
      kv = q16 + kGenRows * LD;
      st = reinterpret_cast<float*>(q16 + (kGenRows + kGenKeys) * LD);
    } else {
      LD = generic_row_len(D);
      qv = gsm;
      kv = gsm + kGenRows * LD;
      st = gsm + (kGenRows + kGenKeys) * LD;
    }
  }
  __device__ float* map_row() const { return st + kGenRows * (kGenKeys + 1); }
  __device__ void stage(bool q, const void* base, int64_t stride, int row0, int n) const {
    const int rows = q ? kGenRows : kGenKeys;
    if constexpr (MF)
      stage_rows16(reinterpret_cast<uint16_t*>(q ? qv : kv), base, stride, row0, n, rows, D);
    else
      stage_rows<IT>(reinterpret_cast<float*>(q ? qv : kv), base, stride, row0, n, rows, D, LD);
  }
  __device__ void score() const {
    if constexpr (MF)
      score_tile16<IT>(reinterpret_cast<const uint16_t*>(qv), reinterpret_cast<const uint16_t*>(kv), st, D);
    else
      score_tile(reinterpret_cast<const float*>(qv), reinterpret_cast<const float*>(kv), st, LD);
  }
};

// Combine over the four consecutive lanes that share a row.
__device__ __forceinline__ float quad_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 1, 64));
  return fmaxf(x, __shfl_xor(x, 2, 64));
}
__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 1, 64);
  return x + __shfl_xor(x, 2, 64);
}

// ------------------------------------------------------------------------------------
// Exact block mass, in the log2 domain (exp(x) = exp2(x * log2 e)).  Pass 1: per row the
// maximum m of s * scale * log2 e and the denominator l = sum exp2(.. - m), tile by tile
// (rescaled when m moves).  Pass 2: each row's per-block sums of exp2(.. - m), divided by
// l, go into the query block's map row; the map is then divided by the block's row count.
// ------------------------------------------------------------------------------------
template <int IT, bool MF>
__global__ __launch_bounds__(256) void block_mass_generic_kernel(PoolArgs a) {
  extern __shared__ float gsm[];
  const int bs = a.bs, nkb = a.nkb;
  const GenTiles<IT, MF> tl(gsm, a.D);
  const float* St = tl.st;
  float* acc = tl.map_row();
  const int qb = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H, h = bh - b * a.H;
  const char* qbase = (const char*)a.q + ((int64_t)b * a.qs[0] + (int64_t)h * a.qs[1]) * ElemSize<IT>::value;
  const char* kbase = (const char*)a.k + ((int64_t)b * a.ks[0] + (int64_t)h * a.ks[1]) * ElemSize<IT>::value;
  const int row_begin = qb * bs, nr = min(bs, a.Nq - row_begin);
  const float c2 = a.scale * kLog2e;
  const int r = threadIdx.x >> 2, qq = threadIdx.x & 3;  // row and key quarter in the walks
  for (int kb = threadIdx.x; kb < nkb; kb += blockDim.x) acc[kb] = 0.f;

  for (int g0 = 0; g0 < nr; g0 += kGenRows) {
    const int ng = min(kGenRows, nr - g0);
    __syncthreads();
    tl.stage(true, qbase, a.qs[2], row_begin + g0, ng);
    float m = neg_inf(), l = 0.f;
    for (int pass = 0; pass < 2; ++pass) {
      int cur_kb = -1, cur_end = 0;  // key block being summed and its end key
      float cur = 0.f;
      for (int k0 = 0; k0 < a.Nk; k0 += kGenKeys) {
        const int nk = min(kGenKeys, a.Nk - k0);
        __syncthreads();  // the previous tile's walk is done with St and Ks
        tl.stage(false, kbase, a.ks[2], k0, nk);
        __syncthreads();
        tl.score();
        __syncthreads();
        if (r < ng) {
          const float* srow = St + r * (kGenKeys + 1);
          const int j0 = 16 * qq, j1 = min(j0 + 16, nk);
          if (pass == 0) {
            float mt = neg_inf();
            for (int j = j0; j < j1; ++j) mt = fmaxf(mt, srow[j] * c2);
            mt = quad_max(mt);
            if (mt > m) {
              l *= fast_exp2(m - mt);
              m = mt;
            }
            float ts = 0.f;
            for (int j = j0; j < j1; ++j) ts += fast_exp2(__builtin_fmaf(srow[j], c2, -m));
            l += quad_sum(ts);
          } else {
            for (int j = j0; j < j1; ++j) {
              const int key = k0 + j;
              if (key >= cur_end) {
                if (cur_kb >= 0) atomicAdd(&acc[cur_kb], cur / l);
                cur_kb = key / bs;
                cur_end = (cur_kb + 1) * bs;
                cur = 0.f;
              }
              cur += fast_exp2(__builtin_fmaf(srow[j], c2, -m));
            }
          }
        }
      }
      if (pass == 1 && r < ng && cur_kb >= 0) atomicAdd(&acc[cur_kb], cur / l);
    }
  }
  __syncthreads();
  float* out = reinterpret_cast<float*>(a.out) + ((int64_t)bh * a.nqb + qb) * nkb;
  for (int kb = threadIdx.x; kb < nkb; kb += blockDim.x) out[kb] = acc[kb] / (float)nr;
}

// ------------------------------------------------------------------------------------
// Max-pool map.  Pass 1: per row m = max_j s_j * sm_scale * log2e.  Pass 2: per (row, key
// block) R = q.dtype(max_j s_j * sm_scale * log2e), and the map entry is the maximum over
// the block's rows of exp2(R - m); the row is then normalised in q.dtype
// (pooling_kernel.py:39-48,65-75,243-244).  A block's keys may be split over the four
// threads of a row and over tiles: each part's maximum goes through the same rounding and
// exp2 and the parts meet in an atomic maximum (both are monotone, so the result is that
// of the whole block).  Causal: key blocks after the query block are skipped and the
// diagonal block adds -1e6 to raw scores above the diagonal.
// ------------------------------------------------------------------------------------
template <int IT, bool MF>
__global__ __launch_bounds__(256) void max_pool_generic_kernel(PoolArgs a) {
  extern __shared__ float gsm[];
  const int bs = a.bs, nkb = a.nkb;
  const GenTiles<IT, MF> tl(gsm, a.D);
  const float* St = tl.st;
  float* acc = tl.map_row();
  unsigned* acc_bits = reinterpret_cast<unsigned*>(acc);
  const int qb = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H, h = bh - b * a.H, hk = h / (a.H / a.Hk);
  const char* qbase = (const char*)a.q + ((int64_t)b * a.qs[0] + (int64_t)h * a.qs[1]) * ElemSize<IT>::value;
  const char* kbase = (const char*)a.k + ((int64_t)b * a.ks[0] + (int64_t)hk * a.ks[1]) * ElemSize<IT>::value;
  const int row_begin = qb * bs, nr = min(bs, a.Nq - row_begin);
  const int kb_end = a.causal ? min(nkb, qb + 1) : nkb;
  const int key_end = min(a.Nk, kb_end * bs);
  // The reference forms qk_scale = fp32(sm_scale) * fp32(1.44269504).
  const float c = a.scale * 1.44269504f;
  const int r = threadIdx.x >> 2, qq = threadIdx.x & 3;
  for (int kb = threadIdx.x; kb < nkb; kb += blockDim.x) acc[kb] = 0.f;

  for (int g0 = 0; g0 < nr; g0 += kGenRows) {
    const int ng = min(kGenRows, nr - g0);
    __syncthreads();
    tl.stage(true, qbase, a.qs[2], row_begin + g0, ng);
    const int qrow = row_begin + g0 + r;
    // causal: the diagonal block's keys above the row get -1e6
    const int diag_lo = a.causal ? max(qb * bs, qrow + 1) : key_end;
    const int diag_hi = a.causal ? (qb + 1) * bs : key_end;
    float m = neg_inf();
    for (int pass = 0; pass < 2; ++pass) {
      int cur_kb = -1, cur_end = 0;
      float cur = neg_inf();
      for (int k0 = 0; k0 < key_end; k0 += kGenKeys) {
        const int nk = min(kGenKeys, key_end - k0);
        __syncthreads();
        tl.stage(false, kbase, a.ks[2], k0, nk);
        __syncthreads();
        tl.score();
        __syncthreads();
        if (r < ng) {
          const float* srow = St + r * (kGenKeys + 1);
          const int j0 = 16 * qq, j1 = min(j0 + 16, nk);
          if (pass == 0) {
            float mt = neg_inf();
            for (int j = j0; j < j1; ++j) {
              const int key = k0 + j;
              const float s = srow[j] + ((key >= diag_lo && key < diag_hi) ? -1.0e6f : 0.f);
              mt = fmaxf(mt, s * c);
            }
            m = fmaxf(m, quad_max(mt));
          } else {
            for (int j = j0; j < j1; ++j) {
              const int key = k0 + j;
              const float s = srow[j] + ((key >= diag_lo && key < diag_hi) ? -1.0e6f : 0.f);
              if (key >= cur_end) {
                if (cur_kb >= 0)
                  atomicMax(&acc_bits[cur_kb], __float_as_uint(fast_exp2(round_elem<IT>(cur * c) - m)));
                cur_kb = key / bs;
                cur_end = (cur_kb + 1) * bs;
                cur = neg_inf();
              }
              cur = fmaxf(cur, s);
            }
          }
        }
      }
      if (pass == 1 && r < ng && cur_kb >= 0)
        atomicMax(&acc_bits[cur_kb], __float_as_uint(fast_exp2(round_elem<IT>(cur * c) - m)));
    }
  }
  __syncthreads();
  // Po in q.dtype, its row sum (fp32 accumulation, rounded to q.dtype), then the division.
  for (int kb = threadIdx.x; kb < nkb; kb += blockDim.x) acc[kb] = kb < kb_end ? round_elem<IT>(acc[kb]) : 0.f;
  __syncthreads();
  __shared__ float part[4];
  float sum = 0.f;
  for (int kb = threadIdx.x; kb < nkb; kb += blockDim.x) sum += acc[kb];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = sum;
  __syncthreads();
  const float total = round_elem<IT>((part[0] + part[1]) + (part[2] + part[3]));
  const int64_t base = ((int64_t)bh * a.nqb + qb) * nkb;
  for (int kb = threadIdx.x; kb < nkb; kb += blockDim.x) {
    const float v = round_elem<IT>(acc[kb] / total);
    if constexpr (IT == kF32) reinterpret_cast<float*>(a.out)[base + kb] = v;
    else reinterpret_cast<uint16_t*>(a.out)[base + kb] = (uint16_t)(pack2<IT>(v, 0.f) & 0xffffu);
  }
}

// The matrix-core path takes 16-bit inputs with a head dim that is a multiple of 16.
static bool generic_mf(int D, int dtype) { return dtype != kF32 && D % 16 == 0; }

size_t generic_pool_lds_need(int D, int nkb, int dtype) {
  return generic_pool_lds_bytes(D, nkb, generic_mf(D, dtype));
}

template <typename Kern>
static hipError_t launch_generic(Kern kern, const PoolArgs& a, bool mf, hipStream_t stream) {
  const dim3 grid(a.nqb, a.B * a.H);
  const size_t lds = generic_pool_lds_bytes(a.D, a.nkb, mf);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  kern<<<grid, 256, lds, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_block_mass_generic(const PoolArgs& a, int dtype, hipStream_t stream) {
  if (a.B * a.H * a.nqb == 0) return hipSuccess;
  const bool mf = generic_mf(a.D, dtype);
  if (dtype == kBF16)
    return mf ? launch_generic(block_mass_generic_kernel<kBF16, true>, a, true, stream)
              : launch_generic(block_mass_generic_kernel<kBF16, false>, a, false, stream);
  if (dtype == kF16)
    return mf ? launch_generic(block_mass_generic_kernel<kF16, true>, a, true, stream)
              : launch_generic(block_mass_generic_kernel<kF16, false>, a, false, stream);
  return launch_generic(block_mass_generic_kernel<kF32, false>, a, false, stream);
}

hipError_t launch_max_pool_generic(const PoolArgs& a, int dtype, hipStream_t stream) {
  if (a.B * a.H * a.nqb == 0) return hipSuccess;
  const bool mf = generic_mf(a.D, dtype);
  if (dtype == kBF16)
    return mf ? launch_generic(max_pool_generic_kernel<kBF16, true>, a, true, stream)
              : launch_generic(max_pool_generic_kernel<kBF16, false>, a, false, stream);
  if (dtype == kF16)
    return mf ? launch_generic(max_pool_generic_kernel<kF16, true>, a, true, stream)
              : launch_generic(max_pool_generic_kernel<kF16, false>, a, false, stream);
  return launch_generic(max_pool_generic_kernel<kF32, false>, a, false, stream);
}

}  // namespace sa
