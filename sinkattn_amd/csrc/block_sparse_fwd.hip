// Block-sparse flash-attention forward for gfx950 (CDNA4).
//
// Semantics follow the call site of the reference's external kernel,
// `_block_sparse_attn` (sinkattention/sparse_attention.py:710-776): 128x128 tiles, the
// listed key blocks of each query block are attended, keys >= Nk are masked, softmax
// scale defaults to 1/sqrt(D), lse is the natural-log row log-sum-exp.
//
// Work decomposition: one 256-thread work-group (4 waves) per (b, h, q-block); wave w
// owns query rows [32w, 32w+32) of the block.  For every listed key block the group
// stages K (row-major) and V^T (transposed while staging) in LDS, then each wave runs
//     S^T = K Q^T          v_mfma_f32_32x32x16 (A = K rows from LDS, B = Q^T in VGPRs)
//     online softmax       exp2 domain, fp32
//     O^T += V^T P^T       (A = V^T rows from LDS, B = P^T straight from the S^T VGPRs)
// Computing the transposed products makes the S^T accumulator layout (one query column
// per lane, keys down the registers) line up with the B-operand layout of the second
// MFMA, so P never leaves registers.  The K rows fed as A operand are permuted (bits 2
// and 3 of the row index swapped) so that the key order in the P^T registers is the
// natural order and every V^T A-operand read is one 16-byte LDS load.

#include "common.h"
#include "kernels.h"
#include "tile.h"

namespace sa {

template <int IT, int CT, int D>
__global__ __launch_bounds__(256) void block_sparse_fwd_kernel(FwdArgs a) {
  constexpr int ES = ElemSize<IT>::value;
  constexpr int KC = D / 8;   // 16-byte chunks per staged K row
  constexpr int DS = D / 16;  // k-steps of the QK^T contraction
  constexpr int DT = D / 32;  // 32-row tiles of O^T
  __shared__ u32x4 lds_k[128 * KC];
  __shared__ u32x4 lds_v[D * 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;

  const int item = a.order ? a.order[blockIdx.x] : (int)blockIdx.x;
  const int bh = item / a.nqb;
  const int qb = item - bh * a.nqb;
  const int b = bh / a.H, h = bh - b * a.H;
  const int cnt = a.counts[item];
  const int32_t* list = a.idx + (int64_t)item * a.nkb;

  const char* qbase = (const char*)a.q + ((int64_t)b * a.qs[0] + (int64_t)h * a.qs[1]) * ES;
  const char* kbase = (const char*)a.k + ((int64_t)b * a.ks[0] + (int64_t)h * a.ks[1]) * ES;
  const char* vbase = (const char*)a.v + ((int64_t)b * a.vs[0] + (int64_t)h * a.vs[1]) * ES;

  const int qrow = qb * 128 + wave * 32 + l32;
  u32x4 qf[DS];
  load_q_operand<IT, CT, D>(qf, qbase, a.qs[2], qrow, a.Nq, hl);

  f32x16 o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = f32x16{};
  float m_run = neg_inf();
  float l_run = 0.f;
  const float c = a.scale * kLog2e;

  const int prow = k_row_perm(l32);
  const int fk = k_swz(prow);

  for (int it = 0; it < cnt; ++it) {
    const int kb = list[it];
    const int key0 = kb * 128;
    __syncthreads();
    stage_k_tile<IT, CT, D, 256>(lds_k, kbase, a.ks[2], key0, a.Nk, tid);
    // Stage V^T: each thread gathers a d-pair of 8 consecutive keys.
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      const int id = i * 256 + tid;
      const int dp = id % (D / 2), kg = id / (D / 2);
      uint32_t w[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = key0 + kg * 8 + e;
        w[e] = key < a.Nk ? load2<IT, CT>(vbase + ((int64_t)key * a.vs[2] + 2 * dp) * ES) : 0u;
      }
      u32x4 ev, od;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ev[j] = (w[2 * j] & 0xffffu) | (w[2 * j + 1] << 16);
        od[j] = (w[2 * j] >> 16) | (w[2 * j + 1] & 0xffff0000u);
      }
      const int d0 = 2 * dp;
      lds_v[d0 * 16 + (kg ^ v_swz(d0))] = ev;
      lds_v[(d0 + 1) * 16 + (kg ^ v_swz(d0 + 1))] = od;
    }
    __syncthreads();

    // S^T tile: 4 sub-tiles of 32 keys x 32 queries.
    f32x16 s[4];
    qk_tile<CT, D>(lds_k, qf, prow, fk, hl, s);
    if (key0 + 128 > a.Nk) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (key0 + t * 32 + tile_key(hl, j) >= a.Nk) s[t][j] = neg_inf();
    }
    float mx = neg_inf();
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[t][j]);
    mx = fmaxf(mx, xor32(mx));
    const float m_new = fmaxf(m_run, mx * c);
    const float alpha = fast_exp2(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int i = 0; i < DT; ++i) o[i] *= alpha;
    u32x4 p[4][2];
    float lsum = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float v0 = fast_exp2(__builtin_fmaf(s[t][8 * u + 2 * e], c, -m_new));
          const float v1 = fast_exp2(__builtin_fmaf(s[t][8 * u + 2 * e + 1], c, -m_new));
          lsum += v0 + v1;
          p[t][u][e] = pack2<CT>(v0, v1);
        }
    l_run += lsum;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int R = dt * 32 + l32;
      const int fv = v_swz(R);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const u32x4 av = lds_v[R * 16 + ((4 * t + 2 * u + hl) ^ fv)];
          o[dt] = mfma32x32x16<CT>(av, p[t][u], o[dt]);
        }
    }
  }

  const float l = l_run + xor32(l_run);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (qrow < a.Nq) {
    char* obase = (char*)a.out +
                  ((int64_t)b * a.os[0] + (int64_t)h * a.os[1] + (int64_t)qrow * a.os[2]) * ES;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = dt * 32 + 8 * g + 4 * hl;
        store4<IT>(obase + (int64_t)d * ES, o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv,
                   o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv);
      }
    if (a.lse != nullptr && hl == 0)
      a.lse[((int64_t)b * a.H + h) * a.Nq + qrow] =
          cnt > 0 ? (m_run + __log2f(l)) * kLn2 : pos_inf();
  }
}

// One wave per (b, h, q-block) row: ballot-compact the mask row into an ascending list.
__global__ __launch_bounds__(256) void plan_rows_kernel(PlanArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= a.rows) return;
  const int qb = row % a.nqb;
  const int bh = row / a.nqb;
  const int h = bh % a.H, b = bh / a.H;
  const uint8_t* m = a.mask + (int64_t)b * a.ms[0] + (int64_t)h * a.ms[1] + (int64_t)qb * a.ms[2];
  int32_t* out = a.idx + (int64_t)row * a.nkb;
  int base = 0;
  for (int c0 = 0; c0 < a.nkb; c0 += 64) {
    const int kb = c0 + lane;
    const bool on = kb < a.nkb && m[(int64_t)kb * a.ms[3]] != 0;
    const uint64_t bal = __ballot(on);
    if (on) out[base + __popcll(bal & ((1ull << lane) - 1ull))] = kb;
    base += __popcll(bal);
  }
  if (lane == 0) a.counts[row] = base;
}

// Single work-group counting sort of rows by descending count.
__global__ __launch_bounds__(1024) void plan_order_kernel(PlanArgs a) {
  extern __shared__ int hist[];  // nkb + 1 bins
  const int tid = threadIdx.x;
  for (int i = tid; i <= a.nkb; i += blockDim.x) hist[i] = 0;
  __syncthreads();
  for (int i = tid; i < a.rows; i += blockDim.x) atomicAdd(&hist[a.counts[i]], 1);
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int c = a.nkb; c >= 0; --c) {
      const int n = hist[c];
      hist[c] = run;
      run += n;
    }
  }
  __syncthreads();
  for (int i = tid; i < a.rows; i += blockDim.x) {
    const int pos = atomicAdd(&hist[a.counts[i]], 1);
    a.order[pos] = i;
  }
}

hipError_t launch_block_sparse_plan(const PlanArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  plan_rows_kernel<<<(a.rows + 3) / 4, 256, 0, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.order == nullptr) return e;
  plan_order_kernel<<<1, 1024, (a.nkb + 1) * sizeof(int), stream>>>(a);
  return hipGetLastError();
}

template <int IT, int CT>
static hipError_t launch_fwd_dt(const FwdArgs& a, int D, hipStream_t stream) {
  const int grid = (int)(a.B * a.H * a.nqb);
  if (D == 128)
    block_sparse_fwd_kernel<IT, CT, 128><<<grid, 256, 0, stream>>>(a);
  else
    block_sparse_fwd_kernel<IT, CT, 64><<<grid, 256, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_block_sparse_fwd(const FwdArgs& a, int dtype, int D, hipStream_t stream) {
  if (a.B * a.H * a.nqb == 0) return hipSuccess;
  switch (dtype) {
    case kBF16: return launch_fwd_dt<kBF16, kBF16>(a, D, stream);
    case kF16: return launch_fwd_dt<kF16, kF16>(a, D, stream);
    default: return launch_fwd_dt<kF32, kBF16>(a, D, stream);
  }
}

}  // namespace sa
