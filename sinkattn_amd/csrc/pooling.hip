// Block-score ("pooling") kernels for gfx950.
//
// block_mass_pool: the reference's exact mode, `_compute_exact_block_mass_scores`
//   (sinkattention/sparse_attention.py:145-227), in one pass over K with no N x N
//   intermediate.  A work-group owns one q-block (128 rows) at a time.  For every key tile
//   it computes S^T with the matrix cores and turns each row's scores into exp2 terms
//   relative to a per-row reference maximum.
//   * bf16/f16 (block_mass_persistent_kernel): persistent groups; the per-(row, key-block)
//     sums go to the group's slot ws[kb][row] of a global workspace.  The reference maximum
//     is the row maximum of the first tile and moves only when a tile's sum exceeds 2^64
//     (kSumLimit); then the row's earlier sums are rescaled.
//   * fp32 (block_mass_f32_kernel): one group per q-block; the sums stay in LDS, and the
//     reference maximum moves when a tile's maximum exceeds it by more than
//     kRescaleMargin (log2 units), rescaling the earlier sums.
//   At the end every row is normalised by its own total and the rows are averaged per key
//   block.
//
// max_pool: `attn_with_pooling` (sinkattention/pooling_kernel.py:11-248) without the
//   [B,H,N,nd] scratch: the per-(row, key-block) maxima of the rows in flight go to the
//   group's slot ws[kb][row] of a global workspace (max_pool_persistent_kernel).
//
// mean_pool: `_compute_pooled_qk_block_scores`' mean branch
//   (sinkattention/sparse_attention.py:79-94,138-142).

#include "common.h"
#include "kernels.h"
#include "tile.h"

namespace sa {

constexpr float kRescaleMargin = 8.f;  // block_mass_f32_kernel only

// ------------------------------------------------------------------------------------
// Exact block mass, 16-bit inputs, head dim 128, block size KB in {16, 32, 64, 128};
// persistent work-groups (up to 3 per CU).
// Each work-group walks items of 128 query rows (128 / KB q-blocks of the map); per item it
// streams every 128-key K tile into LDS by buffer DMA (rows >= Nk read as zero and are
// masked), computes S^T for its 128 rows with the matrix cores and writes each row's sum
// of exp2(scale*log2e*s - m_ref) over every KB-key block of the tile to its private
// workspace slot ws[kb][row] (kb in KB units).  m_ref is the row maximum of the first tile;
// it only moves (and the row's earlier sums are rescaled) if a tile's sum overflows 2^64,
// i.e. when scores rise more than ~64 log2 units above it.  The item's epilogue normalises
// every row by its total and averages the rows of each q-block per key block.
// Key of register j of a lane of 32-key group t, within the group: tile_key(hl, j) =
// (j & 3) + 4 ((j >> 2) & 1) + 8 hl + 16 (j >> 3), so the KB-key block of (t, j) does not
// depend on the lane: t / (KB / 32) for KB >= 32, 2 t + (j >> 3) for KB = 16 (the lane pair
// holds its two 8-key halves).
// ------------------------------------------------------------------------------------
constexpr float kSumLimit = 1.8446744073709552e19f;  // 2^64

template <int KB>
__device__ __forceinline__ constexpr int sub_block(int t, int j) {
  return KB == 16 ? 2 * t + (j >> 3) : (t * 32) / KB;
}

template <int CT, int KB>
__global__ __launch_bounds__(256, 3) void block_mass_persistent_kernel(PoolArgs a, int items) {
  constexpr int DS = 8;
  constexpr int NS = 128 / KB;  // key blocks per 128-key tile, q-blocks per 128-row item
  __shared__ u32x4 lds_k[2048];
  __shared__ float row_inv[128];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5, l32 = lane & 31;
  const int nkb = a.nkb;                 // key blocks of the map (KB keys each)
  const int ntiles = (a.Nk + 127) >> 7;  // 128-key tiles
  const int nqi = (a.Nq + 127) >> 7;     // 128-row items per head
  float* ws = a.ws + (size_t)blockIdx.x * (size_t)nkb * 128;
  const uint32_t kstride = (uint32_t)a.ks[2] * 2;
  const int drow = 4 * wave + (lane >> 4);
  const uint32_t k_off = (uint32_t)drow * kstride + (uint32_t)(((lane & 15) ^ (drow & 15)) * 16);
  const int prow = k_row_perm(l32);
  uint32_t ka[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) ka[ds] = (uint32_t)(prow * 256 + (((2 * ds + hl) ^ (prow & 15)) * 16));
  SA_LDS char* lk = (SA_LDS char*)lds_k;
  const float c = a.scale * kLog2e;
  const int r = wave * 32 + l32;

  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const int bh = item / nqi;
    const int qi = item - bh * nqi;
    const int b = bh / a.H, h = bh - b * a.H;
    const char* qbase = (const char*)a.q + ((int64_t)b * a.qs[0] + (int64_t)h * a.qs[1]) * 2;
    const char* kbase = (const char*)a.k + ((int64_t)b * a.ks[0] + (int64_t)h * a.ks[1]) * 2;
    const int qrow = qi * 128 + r;
    u32x4 qf[DS];
    load_q_operand<CT, CT, 128>(qf, qbase, a.qs[2], qrow, a.Nq, hl);
    float m_ref = neg_inf();
    float l_tot = 0.f;

    for (int kt = 0; kt < ntiles; ++kt) {
      const int key0 = kt * 128;
      __syncthreads();  // the previous tile (or item epilogue) is done with lds_k
      {
        const __amdgpu_buffer_rsrc_t rs =
            make_rsrc(kbase + (int64_t)key0 * kstride, (uint32_t)(a.Nk - key0) * kstride);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          dma16(rs, (SA_LDS void*)(lk + (256 * j + 64 * wave) * 16), k_off + (uint32_t)j * 16u * kstride);
      }
      __syncthreads();  // waits for this group's DMA
      f32x16 s[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) s[t] = f32x16{};
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const u32x4 av = *(SA_LDS const u32x4*)(lk + ka[ds] + t * 8192);
          s[t] = mfma32x32x16<CT>(av, qf[ds], s[t]);
        }
      if (key0 + 128 > a.Nk) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (key0 + t * 32 + tile_key(hl, j) >= a.Nk) s[t][j] = neg_inf();
      }
      if (kt == 0) {  // reference maximum from the first tile (key 0 always exists)
        float mx = neg_inf();
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[t][j]);
        m_ref = max_xor32(mx) * c;
      }
      float ps[NS];
      auto sums = [&]() {
#pragma unroll
        for (int i = 0; i < NS; ++i) ps[i] = 0.f;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int j = 0; j < 16; ++j) ps[sub_block<KB>(t, j)] += fast_exp2(__builtin_fmaf(s[t][j], c, -m_ref));
#pragma unroll
        for (int i = 0; i < NS; ++i) ps[i] = sum_xor32(ps[i]);
      };
      sums();
      float tot = 0.f;
#pragma unroll
      for (int i = 0; i < NS; ++i) tot += ps[i];
      if (!(tot <= kSumLimit)) {
        // Rare: scores far above m_ref.  Move m_ref to this tile's maximum and rescale
        // the row's earlier sums (the two lanes of the row split them by parity).
        float mx = neg_inf();
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[t][j]);
        mx = max_xor32(mx) * c;
        const float f = fast_exp2(m_ref - mx);
        for (int j = hl; j < kt * NS; j += 2) ws[j * 128 + r] *= f;
        l_tot *= f;
        m_ref = mx;
        sums();
        tot = 0.f;
#pragma unroll
        for (int i = 0; i < NS; ++i) tot += ps[i];
      }
      l_tot += tot;
      // the lanes of a row split the stores: lane half hl stores key blocks i = hl (mod 2)
#pragma unroll
      for (int i = 0; i < NS; ++i)
        if ((NS == 1 ? hl == 0 : (i & 1) == hl) && kt * NS + i < nkb) ws[(kt * NS + i) * 128 + r] = ps[i];
    }

    // Epilogue: out[qb][kb] = mean over the q-block's rows of ws[kb][row] / total(row); lane l
    // holds rows l and l + 64, so a q-block of KB rows is one group of KB lanes (KB < 64) or
    // a whole half (KB = 64) or both halves (KB = 128).
    if (hl == 0) row_inv[r] = (qrow < a.Nq) ? 1.f / fmaxf(l_tot, 1e-6f) : 0.f;
    __syncthreads();
    const float inv0 = row_inv[lane], inv1 = row_inv[lane + 64];
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(ws, (uint32_t)nkb * 512u);
    float* out = reinterpret_cast<float*>(a.out);
    for (int kb = wave; kb < nkb; kb += 4) {
      // coherent (L1-bypassing) loads of values other waves of the group wrote
      const float x0 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wrs, (uint32_t)(kb * 512 + lane * 4), 0, 1));
      const float x1 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wrs, (uint32_t)(kb * 512 + lane * 4 + 256), 0, 1));
      float v0 = x0 * inv0, v1 = x1 * inv1;
      if constexpr (KB == 128) {
        v0 += v1;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v0 += __shfl_xor(v0, off, 64);
      } else {
#pragma unroll
        for (int off = (KB >= 64 ? 32 : KB / 2); off >= 1; off >>= 1) {
          v0 += __shfl_xor(v0, off, 64);
          v1 += __shfl_xor(v1, off, 64);
        }
      }
      if (lane % (KB >= 64 ? 64 : KB) == 0) {
        const int g = lane / (KB >= 64 ? 64 : KB);  // q-block of the first half
#pragma unroll
        for (int half = 0; half < (KB == 128 ? 1 : 2); ++half) {
          const int qs = half * (NS / 2 > 0 ? NS / 2 : 1) + g;  // q-block within the item
          const int qb = qi * NS + qs;
          const int rows = min(KB, a.Nq - qb * KB);
          if (qb < a.nqb && rows > 0)
            out[((int64_t)bh * a.nqb + qb) * nkb + kb] = (half == 0 ? v0 : v1) / (float)rows;
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------------
// Exact block mass, f32 inputs: fp32 matrix cores (v_mfma_f32_32x32x2_f32).
// Work-group = 4 waves = 128 rows.  Each 128-key block is staged as four 32-key fp32
// sub-tiles (rows padded to 132 floats).  The contraction index of MFMA step s is
// d = s for lanes 0-31 and d = s + 64 for lanes 32-63, so four consecutive steps read
// one 16-byte LDS vector.
// ------------------------------------------------------------------------------------
template <int NKBMAX>
__global__ __launch_bounds__(256) void block_mass_f32_kernel(PoolArgs a) {
  constexpr int KP = 132;  // padded row length (floats)
  __shared__ float lds_k[32 * KP];
  __shared__ float sums[128 * NKBMAX];
  __shared__ float row_tot[128];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int qb = blockIdx.x;
  const int bh = blockIdx.y;
  const int b = bh / a.H, h = bh - b * a.H;
  const int nkb = a.nkb;

  const float* qbase = (const float*)a.q + ((int64_t)b * a.qs[0] + (int64_t)h * a.qs[1]);
  const float* kbase = (const float*)a.k + ((int64_t)b * a.ks[0] + (int64_t)h * a.ks[1]);

  const int r = wave * 32 + l32;
  const int qrow = qb * 128 + r;
  float qf[64];
#pragma unroll
  for (int s4 = 0; s4 < 16; ++s4) {
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    if (qrow < a.Nq)
      v = *reinterpret_cast<const f32x4*>(qbase + (int64_t)qrow * a.qs[2] + hl * 64 + s4 * 4);
    qf[4 * s4] = v[0]; qf[4 * s4 + 1] = v[1]; qf[4 * s4 + 2] = v[2]; qf[4 * s4 + 3] = v[3];
  }

  const float c = a.scale * kLog2e;
  float m_ref = neg_inf();
  float* my = sums + r * NKBMAX;

  for (int kb = 0; kb < nkb; ++kb) {
    float ps = 0.f;
    for (int t = 0; t < 4; ++t) {
      const int key0 = kb * 128 + t * 32;
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 32 * 32 / 256; ++i) {
        const int id = i * 256 + tid;
        const int row = id >> 5, c4 = id & 31;
        const int key = key0 + row;
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
        if (key < a.Nk) v = *reinterpret_cast<const f32x4*>(kbase + (int64_t)key * a.ks[2] + c4 * 4);
        *reinterpret_cast<f32x4*>(lds_k + row * KP + c4 * 4) = v;
      }
      __syncthreads();
      f32x16 s = f32x16{};
#pragma unroll
      for (int s4 = 0; s4 < 16; ++s4) {
        const f32x4 av = *reinterpret_cast<const f32x4*>(lds_k + l32 * KP + hl * 64 + s4 * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          s = __builtin_amdgcn_mfma_f32_32x32x2f32(av[e], qf[4 * s4 + e], s, 0, 0, 0);
      }
      if (key0 + 32 > a.Nk) {
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (key0 + 8 * (j >> 2) + 4 * hl + (j & 3) >= a.Nk) s[j] = neg_inf();
      }
      float mx = neg_inf();
#pragma unroll
      for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[j]);
      mx = max_xor32(mx) * c;
      if (mx > m_ref + kRescaleMargin) {
        const float f = fast_exp2(m_ref - mx);
        for (int j = hl; j < kb; j += 2) my[j] *= f;
        ps *= f;
        m_ref = mx;
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) ps += fast_exp2(__builtin_fmaf(s[j], c, -m_ref));
    }
    ps = sum_xor32(ps);
    if (hl == 0) my[kb] = ps;
  }
  __syncthreads();
  {
    float tot = 0.f;
    for (int j = hl; j < nkb; j += 2) tot += my[j];
    tot = sum_xor32(tot);
    if (hl == 0) row_tot[r] = tot;
  }
  __syncthreads();
  const int nrows = min(128, a.Nq - qb * 128);
  float* out = reinterpret_cast<float*>(a.out) + ((int64_t)bh * a.nqb + qb) * nkb;
  for (int kb = tid; kb < nkb; kb += 256) {
    float acc = 0.f;
    for (int rr = 0; rr < nrows; ++rr) acc += sums[rr * NKBMAX + kb] / fmaxf(row_tot[rr], 1e-6f);
    out[kb] = acc / (float)nrows;
  }
}

// Rounding of an fp32 value to the 16-bit type CT (returned as fp32).
template <int CT>
__device__ __forceinline__ float round_to(float x);
template <>
__device__ __forceinline__ float round_to<kBF16>(float x) {
  return (float)(__bf16)x;
}
template <>
__device__ __forceinline__ float round_to<kF16>(float x) {
  return (float)(_Float16)x;
}

// ------------------------------------------------------------------------------------
// Max-pool map, persistent form (bf16/f16, head dim 128, block size KB in {16, 32, 64,
// 128}): the structure of block_mass_persistent_kernel (items of 128 query rows, K tiles of
// 128 keys by DMA, S^T on the matrix cores) with the block maxima of each row kept in the
// group's workspace slot ws[kb][row] instead of LDS, so four groups (33-37 KB of LDS, 128
// VGPRs each) fit a CU: per tile a group waits for its own copy, and the other three cover
// that wait.  Per tile: R[r,kb] = q.dtype(max_j s * sm_scale * log2e) for each KB-key block
// (raw-score maximum first, then the scale, as pooling_kernel.py:39-48 does), m_r = max
// over kb of the unrounded values.  Epilogue per q-block and kb: Po[kb] = q.dtype(max over
// the block's rows of exp2(R[r,kb] - m_r)), then the row is normalised in q.dtype
// (pooling_kernel.py:65-75, 243-244).  kv head = h / (H / Hk); causal restricts kb <= qb and
// adds -1e6 to the raw scores above the diagonal of the diagonal block.  Block 128 keeps
// the item's column maxima in LDS (nkb <= 1024); smaller blocks keep them after the
// group's slot, in (128 / KB) * nkb floats of the workspace.
// ------------------------------------------------------------------------------------
template <int CT, int KB>
__global__ __launch_bounds__(256, 4) void max_pool_persistent_kernel(PoolArgs a, int items) {
  constexpr int DS = 8;
  constexpr int NS = 128 / KB;  // key blocks per tile, q-blocks per item
  __shared__ u32x4 lds_k[2048];
  __shared__ float row_m[128];
  __shared__ float colmax[KB == 128 ? 1024 : 1];
  __shared__ float total_sh[KB == 128 ? 1 : 4];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5, l32 = lane & 31;
  const int nkb = a.nkb;
  const int ntiles = (a.Nk + 127) >> 7;
  const int nqi = (a.Nq + 127) >> 7;
  float* ws = a.ws + (size_t)blockIdx.x * (size_t)nkb * (128 + (KB == 128 ? 0 : NS));
  float* cm = ws + (size_t)nkb * 128;  // [NS][nkb] column maxima (KB < 128)
  const uint32_t kstride = (uint32_t)a.ks[2] * 2;
  const int drow = 4 * wave + (lane >> 4);
  const uint32_t k_off = (uint32_t)drow * kstride + (uint32_t)(((lane & 15) ^ (drow & 15)) * 16);
  const int prow = k_row_perm(l32);
  // chunk (2ds + hl) ^ (prow & 15) of row prow: the k-step only flips bits 5-7
  const uint32_t ka0 = (uint32_t)(prow * 256 + ((hl ^ (prow & 15)) * 16));
  SA_LDS char* lk = (SA_LDS char*)lds_k;
  // The reference forms qk_scale = fp32(sm_scale) * fp32(1.44269504).
  const float qk_scale = a.scale * 1.44269504f;
  const int r = wave * 32 + l32;

  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const int bh = item / nqi;
    const int qi = item - bh * nqi;
    const int b = bh / a.H, h = bh - b * a.H;
    const int hk = h / (a.H / a.Hk);
    const int kt_end = a.causal ? min(ntiles, qi + 1) : ntiles;
    const int kb_item = a.causal ? min(nkb, (qi + 1) * NS) : nkb;  // key blocks any row of the item sees
    const char* qbase = (const char*)a.q + ((int64_t)b * a.qs[0] + (int64_t)h * a.qs[1]) * 2;
    const char* kbase = (const char*)a.k + ((int64_t)b * a.ks[0] + (int64_t)hk * a.ks[1]) * 2;
    const int qrow = qi * 128 + r;
    const int qbr = qrow / KB;  // this row's q-block
    u32x4 qf[DS];
    load_q_operand<CT, CT, 128>(qf, qbase, a.qs[2], qrow, a.Nq, hl);
    float m = neg_inf();

    for (int kt = 0; kt < kt_end; ++kt) {
      const int key0 = kt * 128;
      __syncthreads();  // the previous tile (or item epilogue) is done with lds_k
      {
        const __amdgpu_buffer_rsrc_t rs =
            make_rsrc(kbase + (int64_t)key0 * kstride, (uint32_t)(a.Nk - key0) * kstride);
#pragma unroll
        for (int j = 0; j < 8; ++j)
          dma16(rs, (SA_LDS void*)(lk + (256 * j + 64 * wave) * 16), k_off + (uint32_t)j * 16u * kstride);
      }
      __syncthreads();  // waits for this group's DMA
      f32x16 s[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) s[t] = f32x16{};
      {
        // Flat step i = 4 ds + t.  The read for step i + 2 is issued right after the MFMA
        // of step i (the scheduling groups pin that order), so each read has two MFMAs to
        // land; a deeper ring does not fit the 128 VGPRs of four groups per CU.
        u32x4 kr[4];
        auto kread = [&](int i) __attribute__((always_inline)) {
          return *(SA_LDS const u32x4*)(lk + (ka0 ^ (32u * (i >> 2))) + (i & 3) * 8192);
        };
        kr[0] = kread(0);
        kr[1] = kread(1);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
        for (int i = 0; i < 4 * DS; ++i) {
          s[i & 3] = mfma32x32x16<CT>(kr[i & 3], qf[i >> 2], s[i & 3]);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (i + 2 < 4 * DS) {
            kr[(i + 2) & 3] = kread(i + 2);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
        }
      }
      const bool diag = a.causal && kt == qi;
      if (key0 + 128 > a.Nk || diag) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int key = key0 + t * 32 + tile_key(hl, j);
            if (diag) {
              const int kbk = key / KB;
              if (kbk == qbr && qrow < key) s[t][j] += -1.0e6f;
              if (kbk > qbr) s[t][j] = neg_inf();  // a key block past the row's own: not seen
            }
            if (key >= a.Nk) s[t][j] = neg_inf();
          }
      }
      float mx[NS];
#pragma unroll
      for (int i = 0; i < NS; ++i) mx[i] = neg_inf();
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) mx[sub_block<KB>(t, j)] = fmaxf(mx[sub_block<KB>(t, j)], s[t][j]);
#pragma unroll
      for (int i = 0; i < NS; ++i) {
        mx[i] = max_xor32(mx[i]) * qk_scale;
        m = fmaxf(m, mx[i]);
        if ((NS == 1 ? hl == 0 : (i & 1) == hl) && kt * NS + i < nkb) ws[(kt * NS + i) * 128 + r] = round_to<CT>(mx[i]);
      }
    }

    // Epilogue.  Rows past the end of the sequence take no part (m = +inf gives 0).
    if (hl == 0) row_m[r] = (qrow < a.Nq) ? m : pos_inf();
    __syncthreads();
    const float m0 = row_m[lane], m1 = row_m[lane + 64];
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(ws, (uint32_t)nkb * 512u);
    if constexpr (KB == 128) {
      for (int kb = wave; kb < kb_item; kb += 4) {
        // coherent (L1-bypassing) loads of values other waves of the group wrote
        const float x0 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wrs, (uint32_t)(kb * 512 + lane * 4), 0, 1));
        const float x1 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wrs, (uint32_t)(kb * 512 + lane * 4 + 256), 0, 1));
        float v = fmaxf(fast_exp2(x0 - m0), fast_exp2(x1 - m1));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
        if (lane == 0) colmax[kb] = round_to<CT>(v);
      }
      __syncthreads();
      // Row normalisation in q.dtype: sum (fp32 accumulate, rounded), then divide.
      if (wave == 0) {
        float part = 0.f;
        for (int kb = lane; kb < kb_item; kb += 64) part += colmax[kb];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
        if (lane == 0) total_sh[0] = round_to<CT>(part);
      }
      __syncthreads();
      const float total = total_sh[0];
      uint16_t* out = reinterpret_cast<uint16_t*>(a.out) + ((int64_t)bh * a.nqb + qi) * nkb;
      for (int kb = tid; kb < nkb; kb += 256) {
        const float v = kb < kb_item ? colmax[kb] / total : 0.f;
        out[kb] = (uint16_t)(pack2<CT>(v, 0.f) & 0xffffu);
      }
    } else {
      // Pass 1: column maxima of every (q-block, key block) of the item into cm[qs][kb]:
      // lane l holds rows l and l + 64, so a q-block is a group of KB lanes (KB < 64) or a
      // whole half (KB = 64).
      constexpr int G = KB >= 64 ? 64 : KB;
      for (int kb = wave; kb < kb_item; kb += 4) {
        const float x0 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wrs, (uint32_t)(kb * 512 + lane * 4), 0, 1));
        const float x1 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wrs, (uint32_t)(kb * 512 + lane * 4 + 256), 0, 1));
        float v0 = fast_exp2(x0 - m0), v1 = fast_exp2(x1 - m1);
#pragma unroll
        for (int off = G / 2; off >= 1; off >>= 1) {
          v0 = fmaxf(v0, __shfl_xor(v0, off, 64));
          v1 = fmaxf(v1, __shfl_xor(v1, off, 64));
        }
        if (lane % G == 0) {
          const int g = lane / G;
          cm[(size_t)g * nkb + kb] = round_to<CT>(v0);
          cm[(size_t)(NS / 2 + g) * nkb + kb] = round_to<CT>(v1);
        }
      }
      __syncthreads();  // the column maxima are in memory (the barrier drains this group's stores)
      // Pass 2: per q-block (one wave each), the row total in q.dtype, then the division.
      const __amdgpu_buffer_rsrc_t crs = make_rsrc(cm, (uint32_t)(NS * nkb) * 4u);
      for (int qs = wave; qs < NS; qs += 4) {
        const int qb = qi * NS + qs;
        if (qb >= a.nqb) continue;
        const int kb_end = a.causal ? min(nkb, qb + 1) : nkb;
        float part = 0.f;
        for (int kb = lane; kb < kb_end; kb += 64)
          part += __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(crs, (uint32_t)((qs * nkb + kb) * 4), 0, 1));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
        const float total = round_to<CT>(part);
        uint16_t* out = reinterpret_cast<uint16_t*>(a.out) + ((int64_t)bh * a.nqb + qb) * nkb;
        for (int kb = lane; kb < nkb; kb += 64) {
          const float cv = kb < kb_end ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                              crs, (uint32_t)((qs * nkb + kb) * 4), 0, 1))
                                       : 0.f;
          out[kb] = (uint16_t)(pack2<CT>(kb < kb_end ? cv / total : 0.f, 0.f) & 0xffffu);
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------------
// Mean-pooled scores.  Pass 1: per-block means of Q and K (replicate-padded tail).
// ------------------------------------------------------------------------------------
template <int IT>
__global__ __launch_bounds__(128) void mean_pool_rows_kernel(PoolArgs a, int which) {
  // blockIdx.x = block index, blockIdx.y = bh; thread = d.
  const int blk = blockIdx.x, bh = blockIdx.y, d = threadIdx.x;
  const int b = bh / a.H, h = bh - b * a.H;
  const int N = which == 0 ? a.Nq : a.Nk;
  const int nb = which == 0 ? a.nqb : a.nkb;
  const int64_t* st = which == 0 ? a.qs : a.ks;
  const void* base = which == 0 ? a.q : a.k;
  const int D = blockDim.x;
  const int bs = a.bs;
  float acc = 0.f;
  for (int i = 0; i < bs; ++i) {
    const int n = min(blk * bs + i, N - 1);
    const int64_t off = (int64_t)b * st[0] + (int64_t)h * st[1] + (int64_t)n * st[2] + d;
    float x;
    if (IT == kF32) x = reinterpret_cast<const float*>(base)[off];
    else if (IT == kBF16) x = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[off]);
    else x = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[off]);
    acc += x;
  }
  float* dst = a.ws + (which == 0 ? 0 : (int64_t)a.B * a.H * a.nqb * D);
  dst[((int64_t)bh * nb + blk) * D + d] = acc / (float)bs;
}

// Pass 2: one wave per (bh, qb) row: dot products against every pooled key, softmax.
__global__ __launch_bounds__(64) void mean_pool_scores_kernel(PoolArgs a, int D) {
  const int qb = blockIdx.x, bh = blockIdx.y, lane = threadIdx.x;
  const float* qp = a.ws + ((int64_t)bh * a.nqb + qb) * D;
  const float* kp = a.ws + (int64_t)a.B * a.H * a.nqb * D + (int64_t)bh * a.nkb * D;
  float* out = reinterpret_cast<float*>(a.out) + ((int64_t)bh * a.nqb + qb) * a.nkb;
  float mx = neg_inf();
  for (int kb = lane; kb < a.nkb; kb += 64) {
    float acc = 0.f;
    for (int d = 0; d < D; ++d) acc = __builtin_fmaf(qp[d], kp[(int64_t)kb * D + d], acc);
    const float sc = acc * a.scale;
    out[kb] = sc;
    mx = fmaxf(mx, sc);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  float sum = 0.f;
  for (int kb = lane; kb < a.nkb; kb += 64) {
    const float e = expf(out[kb] - mx);
    out[kb] = e;
    sum += e;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off, 64);
  for (int kb = lane; kb < a.nkb; kb += 64) out[kb] = out[kb] / sum;
}

// ------------------------------------------------------------------------------------
// Compute units of the current device (256, an MI355X, if the query fails).
int device_cu_count() {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) cus = n;
  }
  return cus;
}

// Resident work-groups of the persistent block-mass kernel on the current device.
int block_mass_groups() { return 3 * device_cu_count(); }
int max_pool_groups() { return 4 * device_cu_count(); }

hipError_t launch_block_mass_pool(const PoolArgs& a, int dtype, int D, hipStream_t stream) {
  (void)D;
  if (a.B * a.H * a.nqb == 0) return hipSuccess;
  const dim3 grid(a.nqb, a.B * a.H);
  if (dtype == kF32) {
    if (a.nkb <= 64) block_mass_f32_kernel<64><<<grid, 256, 0, stream>>>(a);
    else block_mass_f32_kernel<256><<<grid, 256, 0, stream>>>(a);
    return hipGetLastError();
  }
  const int items = a.B * a.H * ((a.Nq + 127) / 128);
  const int groups = min(items, block_mass_groups());
#define SA_MASS(KB)                                                                     \
  do {                                                                                  \
    if (dtype == kBF16)                                                                 \
      block_mass_persistent_kernel<kBF16, KB><<<groups, 256, 0, stream>>>(a, items);    \
    else                                                                                \
      block_mass_persistent_kernel<kF16, KB><<<groups, 256, 0, stream>>>(a, items);     \
  } while (0)
  switch (a.bs) {
    case 16: SA_MASS(16); break;
    case 32: SA_MASS(32); break;
    case 64: SA_MASS(64); break;
    default: SA_MASS(128); break;
  }
#undef SA_MASS
  return hipGetLastError();
}

hipError_t launch_max_pool(const PoolArgs& a, int dtype, int D, hipStream_t stream) {
  (void)D;
  if (a.B * a.H * a.nqb == 0) return hipSuccess;
  const int items = a.B * a.H * ((a.Nq + 127) / 128);
  const int groups = min(items, max_pool_groups());
#define SA_MAXP(KB)                                                                  \
  do {                                                                               \
    if (dtype == kBF16)                                                              \
      max_pool_persistent_kernel<kBF16, KB><<<groups, 256, 0, stream>>>(a, items);   \
    else                                                                             \
      max_pool_persistent_kernel<kF16, KB><<<groups, 256, 0, stream>>>(a, items);    \
  } while (0)
  switch (a.bs) {
    case 16: SA_MAXP(16); break;
    case 32: SA_MAXP(32); break;
    case 64: SA_MAXP(64); break;
    default: SA_MAXP(128); break;
  }
#undef SA_MAXP
  return hipGetLastError();
}

hipError_t launch_mean_pool(const PoolArgs& a, int dtype, int D, hipStream_t stream) {
  if (a.B * a.H == 0) return hipSuccess;
  for (int which = 0; which < 2; ++which) {
    const dim3 grid(which == 0 ? a.nqb : a.nkb, a.B * a.H);
    if (dtype == kF32) mean_pool_rows_kernel<kF32><<<grid, D, 0, stream>>>(a, which);
    else if (dtype == kBF16) mean_pool_rows_kernel<kBF16><<<grid, D, 0, stream>>>(a, which);
    else mean_pool_rows_kernel<kF16><<<grid, D, 0, stream>>>(a, which);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  mean_pool_scores_kernel<<<dim3(a.nqb, a.B * a.H), 64, 0, stream>>>(a, D);
  return hipGetLastError();
}

}  // namespace sa
