// Block-sparse flash-attention forward for gfx950 (CDNA4).
//
// Semantics follow the call site of the reference's external kernel,
// `_block_sparse_attn` (sinkattention/sparse_attention.py:710-776): 128x128 tiles, the
// listed key blocks of each query block are attended, keys >= Nk are masked, softmax
// scale defaults to 1/sqrt(D), lse is the natural-log row log-sum-exp.
//
// Work decomposition: one 256-thread work-group (4 waves) per (b, h, q-block); wave w
// owns query rows [32w, 32w+32) of the block.  For every listed key block the group
// brings K and V into LDS, then each wave runs
//     S^T = K Q^T          (A = K rows from LDS, B = Q^T in VGPRs)
//     online softmax       exp2 domain, fp32
//     O^T += V^T P^T       (A = V^T rows from LDS, B = P^T straight from the S^T VGPRs)
// Computing the transposed products makes the S^T accumulator layout (one query column
// per lane, keys down the registers) line up with the B-operand layout of the second
// MFMA, so P never leaves registers.  block_sparse_fwd_kernel (D = 32 and 64, all input
// types; v_mfma_f32_32x32x16, K rows permuted so that the key order in the P^T registers is
// natural) stages K and V^T through registers, V transposed while staging;
// block_sparse_fwd_d128_kernel (D = 128, 16-bit; v_mfma_f32_16x16x32) copies K and V
// row-major by buffer DMA and reads V^T with transpose loads; block_sparse_fwd_f32_kernel
// splits fp32 operands into bf16 pairs.  The plan kernels at the end of the file turn the
// bool mask into per-row lists and the launch order.

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
  if (item < 0) return;
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
  const int fk = k_swz_kc<D / 8>(prow);

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
    mx = max_xor32(mx);
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

  const float l = sum_xor32(l_run);
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

// ------------------------------------------------------------------------------------
// D = 128, bf16/f16: K and V tiles go global -> LDS by buffer DMA (no staging
// registers; rows >= Nk read as zero through the buffer bounds), and V^T is read from
// the row-major V tile with the gfx950 transpose read ds_read_b64_tr_b16.  Both products
// run on v_mfma_f32_16x16x32, which with random 16-bit operands draws less power per flop
// than 32x32x16, so the power-limited chip holds a higher clock.  A wave's 32 query rows
// are two 16-column tiles qt:
//     S^T[16 kt .. +16, qt] = K Q^T        (A = 16 K rows from LDS, B = Q^T in VGPRs)
//     O^T[16 dt .. +16, qt] += V^T P^T     (A = V^T by transpose reads, B = P^T)
// Lane l holds query 16 qt + l % 16 in both products; its S^T registers (kt, qt) hold keys
// 16 kt + 4 (l / 16) + i, i < 4.  A PV k-step kc of 32 keys takes its eight B values from
// S^T tiles (2 kc, qt) and (2 kc + 1, qt), and the transpose reads pick the same keys for
// the A operand, so P never leaves the registers.  The row sums come from the matrix cores as
// well: one more MFMA per k-step and q tile with an all-ones A operand sums the 16-bit P values
// the PV product uses (O / l is then a weighted mean with weights that sum to one; l is within
// 2^-8 relative of the fp32 sum for bf16, 2^-11 for f16), which keeps 64 adds per tile off
// the VALU.  K and V are staged against each other:
// V(i)'s copies are spread over S(i) and K(i+1)'s over softmax(i), one per step, so that
// the copies of the four waves never queue up at the CU's vector-memory pipe in one burst;
// three work-group barriers per tile (K free, V landed, V free and K(i+1) landed).  LDS
// layout: 128 rows x 16 chunks of 16 bytes per tile, physical chunk = logical ^ (row & 15)
// for K (a 16-lane K read touches 16 distinct chunks) and logical ^ 2 (row & 7) for V (a
// half-wave transpose read touches 8 distinct 32-byte column pairs).
// ------------------------------------------------------------------------------------
constexpr float kLazyRescaleLog2 = 8.0f;

// Per-lane LDS addresses of the d128 tile loop (bytes).
struct D128Lanes {
  uint32_t k_off, v_off;  // global byte offset of this lane's first 16-byte DMA chunk
  uint32_t ka[4];         // K A operand of k-step ks: row l % 16 (+ 16 kt), chunk 4 ks + l / 16
  uint32_t va[8];         // V^T transpose reads of d-tile dt (+ 32 kc rows, + 16 h rows)
};

__device__ __forceinline__ D128Lanes d128_lanes(int wave, int lane, uint32_t kstride, uint32_t vstride) {
  D128Lanes L;
  const int g = lane >> 4, sl = lane & 15;
  // DMA: instruction j of wave w fills tile rows 16j + 4w + lane/16 (LDS bytes
  // [(256j + 64w) * 16, +1024)); the swizzle of those rows does not depend on j.
  const int drow = 4 * wave + g;
  L.k_off = (uint32_t)drow * kstride + (uint32_t)((sl ^ (drow & 15)) * 16);
  L.v_off = (uint32_t)drow * vstride + (uint32_t)((sl ^ (2 * (drow & 7))) * 16);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) L.ka[ks] = (uint32_t)(sl * 256 + (((4 * ks + g) ^ sl) * 16));
  // Transpose read h of d-tile dt at k-step kc: lane s of 16-lane group g points at key row
  // 32 kc + 16 h + 4 g + s / 4, columns 16 dt + 4 (s % 4) .. +3.  Lane l of the group then
  // receives element l % 4 of the rows of lanes 4 j + (l % 16) / 4, j < 4: d = 16 dt + l % 16
  // at keys 32 kc + 16 h + 4 g + j, the keys of B slots 4 h + j.
  const int row = 4 * g + (sl >> 2);  // + 32 kc + 16 h, which leave row & 7 unchanged
  const int a4 = sl & 3;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    const int chunk = 2 * dt + (a4 >> 1);
    L.va[dt] = (uint32_t)(row * 256 + ((chunk ^ (2 * (row & 7))) * 16) + (a4 & 1) * 8);
  }
  return L;
}

// Copy j (of 8) of this wave's share of a 128-row tile: rows 16j + 4w + lane/16, from the
// buffer `rs` (rows past its size read as zero) into the LDS tile at `dst`.
__device__ __forceinline__ void d128_copy_one(SA_LDS char* dst, const __amdgpu_buffer_rsrc_t& rs, uint32_t stride,
                                              uint32_t lane_off, int wave, int j) {
  dma16(rs, (SA_LDS void*)(dst + (256 * j + 64 * wave) * 16), lane_off + (uint32_t)j * 16u * stride);
}

// 128 rows of K (or V) from `base` (row stride `stride` bytes, `rows_valid` rows readable:
// rows past it read as zero through the buffer bounds) into the LDS tile at `dst`.
__device__ __forceinline__ void d128_copy_tile(SA_LDS char* dst, const char* base, uint32_t stride,
                                               int rows_valid, uint32_t lane_off, int wave) {
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(base, (uint32_t)rows_valid * stride);
#pragma unroll
  for (int j = 0; j < 8; ++j) d128_copy_one(dst, rs, stride, lane_off, wave, j);
}

// One 128-key tile of the d128 loop for this wave's 32 query rows:
//   S^T = K Q^T from the K tile, with vcopy(j) (this tile's V copy j into the V buffer, free
//   since the previous tile's B2) after every fourth (k-step, key tile) pair; barrier B1
//   (every wave is done with K); the online softmax with kcopy(j) (the next tile's K copy j
//   into the K buffer) after step j; barrier BV (every wave's V copies have landed: vmcnt(8)
//   leaves only the eight K copies issued after them in flight); O^T += V^T P^T from the V
//   tile; barrier B2 (the next K has landed, every wave is done with V).  kcopy must issue a
//   copy for every j, also after the last tile (then from a 0-byte buffer), so that the
//   count of BV holds.
// Keys at or past klim are masked; bias is added to the log2-domain logits (compensation
// tiles); c = softmax scale * log2(e).  g = lane / 16.
template <int CT, typename FV, typename FK>
__device__ __forceinline__ void d128_tile(SA_LDS char* lk, SA_LDS char* lv, const D128Lanes& L,
                                          const u32x4 (&qf)[2][4], int key0, int klim, float bias,
                                          float c, int g, f32x4 (&o)[8][2], float (&m_run)[2],
                                          f32x4 (&l_acc)[2], FV&& vcopy, FK&& kcopy) {
  constexpr int KR = 4;  // K reads issued ahead of their MFMAs
  constexpr int VR = 3;  // transpose-read pairs issued ahead of their MFMAs
  f32x4 s[8][2];
#pragma unroll
  for (int kt = 0; kt < 8; ++kt) {
    s[kt][0] = f32x4{};
    s[kt][1] = f32x4{};
  }
  {
    // pair p = 8 ks + kt: one K read (rows 16 kt .., d slice ks), the MFMAs of both q tiles
    u32x4 kr[32];
    auto kread = [&](int p) { return *(SA_LDS const u32x4*)(lk + L.ka[p >> 3] + (p & 7) * 4096); };
#pragma unroll
    for (int p = 0; p < KR; ++p) kr[p] = kread(p);
    __builtin_amdgcn_sched_group_barrier(0x100, KR, 0);
#pragma unroll
    for (int p = 0; p < 32; ++p) {
      const int ks = p >> 3, kt = p & 7;
      s[kt][0] = mfma16x16x32<CT>(kr[p], qf[0][ks], s[kt][0]);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (p + KR < 32) {
        kr[p + KR] = kread(p + KR);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      s[kt][1] = mfma16x16x32<CT>(kr[p], qf[1][ks], s[kt][1]);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if ((p & 3) == 3) {
        vcopy(p >> 2);  // V copy of this tile, one per four pairs
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
    }
  }
  // B1: every wave is done reading K (own LDS reads returned); V copies may still fly
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0) only
  __builtin_amdgcn_s_barrier();

  if (key0 + 128 > klim) {
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (key0 + 16 * kt + 4 * g + i >= klim) {
          s[kt][0][i] = neg_inf();
          s[kt][1][i] = neg_inf();
        }
  }
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    float mx = neg_inf();
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[kt][qt][i]);
    mx = max_col16(mx);
    const float m_tile = __builtin_fmaf(mx, c, bias);
    if (m_tile > m_run[qt] + kLazyRescaleLog2) {
      const float alpha = fast_exp2(m_run[qt] - m_tile);
      l_acc[qt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) o[dt][qt] *= alpha;
      m_run[qt] = m_tile;
    }
  }
  u32x4 p[4][2];
  auto make_p = [&](int kc, int qt) {
    const float nb = bias - m_run[qt];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float v0 = fast_exp2(__builtin_fmaf(s[2 * kc + h][qt][2 * e], c, nb));
        const float v1 = fast_exp2(__builtin_fmaf(s[2 * kc + h][qt][2 * e + 1], c, nb));
        p[kc][qt][2 * h + e] = pack2<CT>(v0, v1);
      }
  };
  auto vread = [&](int r) -> u32x4 {  // r = 8 kc + dt
    SA_LDS char* base = lv + L.va[r & 7] + (r >> 3) * 8192;
    const v4i16 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((SA_LDS v4i16*)base);
    const v4i16 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((SA_LDS v4i16*)(base + 4096));
    const u32x2 y0 = __builtin_bit_cast(u32x2, x0), y1 = __builtin_bit_cast(u32x2, x1);
    return u32x4{y0[0], y0[1], y1[0], y1[1]};
  };
  // softmax, with the next tile's K copies spread over its steps
#pragma unroll
  for (int step = 0; step < 8; ++step) {
    make_p(step >> 1, step & 1);
    kcopy(step);
    __builtin_amdgcn_sched_barrier(0);
  }
  // BV: this tile's V has landed for every wave (the own V copies are done once at most the
  // eight K copies issued after them are in flight)
  __builtin_amdgcn_s_waitcnt(8 | (7 << 4) | (15 << 8) | (0 << 14));  // vmcnt(8)
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_s_setprio(1);
  {
    // pair r = 8 kc + dt: two transpose reads (d tile dt, keys of k-step kc), both q tiles
    u32x4 vr[32];
#pragma unroll
    for (int r = 0; r < VR; ++r) vr[r] = vread(r);
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * VR, 0);
#pragma unroll
    for (int r = 0; r < 32; ++r) {
      const int kc = r >> 3, dt = r & 7;
      o[dt][0] = mfma16x16x32<CT>(vr[r], p[kc][0], o[dt][0]);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (r + VR < 32) {
        vr[r + VR] = vread(r + VR);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      o[dt][1] = mfma16x16x32<CT>(vr[r], p[kc][1], o[dt][1]);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (dt == 7) {
        // row sums of the 16-bit P of this k-step: A = all ones, so every row of the product
        // is the column sum, and every lane holds its query's running sum
        const uint32_t one = CT == kBF16 ? 0x3F803F80u : 0x3C003C00u;
        const u32x4 ones = {one, one, one, one};
        l_acc[0] = mfma16x16x32<CT>(ones, p[kc][0], l_acc[0]);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        l_acc[1] = mfma16x16x32<CT>(ones, p[kc][1], l_acc[1]);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
    }
  }
  __builtin_amdgcn_s_setprio(0);
  drain_then_barrier();  // B2: next K landed, every wave done with V
}

// Everything the d128 kernels need to know about one (b, h, q-block) work item.  All values
// are wave-uniform (scalar registers).
struct D128Item {
  int item, qb, cnt, ntot;
  const char *qbase, *kbase, *vbase, *kdbase, *vdbase;
  const SA_CONST int32_t* list;
};

__device__ __forceinline__ D128Item d128_item(const FwdArgs& a, int item) {
  D128Item it;
  it.item = item;
  const int bh = item / a.nqb;
  it.qb = item - bh * a.nqb;
  const int b = bh / a.H, h = bh - b * a.H;
  // The plan is read-only for the kernel's lifetime: read it through the constant
  // address space so the list walk compiles to scalar loads and never enters the
  // vector-memory counter the DMA waits rely on.
  it.cnt = __builtin_amdgcn_readfirstlane(((const SA_CONST int32_t*)a.counts)[item]);
  it.list = (const SA_CONST int32_t*)(a.idx + (int64_t)item * a.nkb);
  // Compensation tiles: after its listed tiles, a q-block below comp_qblocks attends every
  // 128-key tile of kd/vd (same row strides as k/v) with comp_bias added to its logits.
  it.ntot = it.cnt + (it.qb < a.comp_qblocks ? (a.Nd + 127) >> 7 : 0);
  it.qbase = (const char*)a.q + ((int64_t)b * a.qs[0] + (int64_t)h * a.qs[1]) * 2;
  it.kbase = (const char*)a.k + ((int64_t)b * a.ks[0] + (int64_t)h * a.ks[1]) * 2;
  it.vbase = (const char*)a.v + ((int64_t)b * a.vs[0] + (int64_t)h * a.vs[1]) * 2;
  it.kdbase = (const char*)a.kd + ((int64_t)b * a.kds[0] + (int64_t)h * a.kds[1]) * 2;
  it.vdbase = (const char*)a.vd + ((int64_t)b * a.vds[0] + (int64_t)h * a.vds[1]) * 2;
  return it;
}

// Tile `t` of an item's walk (listed tiles, then compensation tiles): its first key.  The
// list entry is read unconditionally at an index clamped into the row's own list, so that the
// load can be issued a whole tile before it is needed without ever leaving the plan.
__device__ __forceinline__ int d128_key0(const D128Item& it, int t) {
  const int e = it.list[t < it.cnt ? t : (it.cnt > 0 ? it.cnt - 1 : 0)];
  return t < it.cnt ? e * 128 : (t - it.cnt) * 128;
}

// K rows [key0, key0 + 128) of the listed keys (comp = false) or of the pooled keys
// (comp = true); rows at or past klim read as zero.
template <int CT>
__device__ __forceinline__ void d128_issue_k(const D128Item& it, int key0, int klim, bool comp, SA_LDS char* lk,
                                             const D128Lanes& L, uint32_t kstride, int wave) {
  const char* base = (comp ? it.kdbase : it.kbase) + (int64_t)key0 * kstride;
  d128_copy_tile(lk, base, kstride, klim - key0, L.k_off, wave);
}

// O of this wave's 32 rows through its 8 KB of an idle LDS tile buffer: lane l holds d values
// 16 dt + 4 (l / 16) .. +3 of row 16 qt + l % 16, written as 8-byte pieces; after the
// transpose every store instruction writes 4 whole 256-byte rows.  The caller guarantees that
// no wave reads the buffer and no copy into it is in flight; each wave touches only its own
// slice.
template <int CT>
__device__ __forceinline__ void d128_store_o_staged(const FwdArgs& a, const D128Item& it, const f32x4 (&o)[8][2],
                                                    const float (&m_run)[2], const f32x4 (&l_acc)[2],
                                                    SA_LDS char* buf, int wave, int lane) {
  const int g = lane >> 4, sl = lane & 15;
  float l[2], inv[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    l[qt] = l_acc[qt][0];
    inv[qt] = l[qt] > 0.f ? 1.f / l[qt] : 0.f;
  }
  SA_LDS char* ob = buf + wave * 8192;
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int chunk = (2 * dt + (g >> 1)) ^ sl;  // row 16 qt + sl: row & 15 == sl
      u32x2 w;
      w[0] = pack2<CT>(o[dt][qt][0] * inv[qt], o[dt][qt][1] * inv[qt]);
      w[1] = pack2<CT>(o[dt][qt][2] * inv[qt], o[dt][qt][3] * inv[qt]);
      *(SA_LDS u32x2*)(ob + (16 * qt + sl) * 256 + chunk * 16 + (g & 1) * 8) = w;
    }
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0) only
  const int bh = it.item / a.nqb;
  const int b = bh / a.H, h = bh - b * a.H;
  const int q0 = it.qb * 128 + wave * 32;
  char* obase = (char*)a.out + ((int64_t)b * a.os[0] + (int64_t)h * a.os[1]) * 2;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int rr = 4 * i + (lane >> 4), cc = lane & 15;
    const u32x4 val = *(SA_LDS const u32x4*)(ob + rr * 256 + ((cc ^ (rr & 15)) * 16));
    if (q0 + rr < a.Nq)
      *reinterpret_cast<u32x4*>(obase + ((int64_t)(q0 + rr) * a.os[2]) * 2 + cc * 16) = val;
  }
  if (a.lse != nullptr && g == 0) {
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      const int qrow = q0 + 16 * qt + sl;
      if (qrow < a.Nq)
        a.lse[((int64_t)b * a.H + h) * a.Nq + qrow] = it.ntot > 0 ? (m_run[qt] + __log2f(l[qt])) * kLn2 : pos_inf();
    }
  }
}

// ------------------------------------------------------------------------------------
// The per-q-block form: one work-group per order slot (or per row without an order).
// ------------------------------------------------------------------------------------
template <int CT>
__global__ __launch_bounds__(256, 2) void block_sparse_fwd_d128_kernel(FwdArgs a) {
  __shared__ u32x4 lds_k[2048];
  __shared__ u32x4 lds_v[2048];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, sl = lane & 15;
  const int item = __builtin_amdgcn_readfirstlane(a.order ? a.order[blockIdx.x] : (int)blockIdx.x);
  if (item < 0) return;
  const D128Item it = d128_item(a, item);
  const uint32_t kstride = (uint32_t)a.ks[2] * 2, vstride = (uint32_t)a.vs[2] * 2;
  const D128Lanes L = d128_lanes(wave, lane, kstride, vstride);
  SA_LDS char* lk = (SA_LDS char*)lds_k;
  SA_LDS char* lv = (SA_LDS char*)lds_v;

  // Q^T B operands: query 16 qt + l % 16 of the wave's rows, d slice 32 ks + 8 (l / 16)
  u32x4 qf[2][4];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int qrow = it.qb * 128 + wave * 32 + 16 * qt + sl;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qf[qt][ks] = qrow < a.Nq ? *(const u32x4*)(it.qbase + ((int64_t)qrow * a.qs[2] + 32 * ks + 8 * g) * 2)
                               : u32x4{0, 0, 0, 0};
  }
  f32x4 o[8][2];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    o[dt][0] = f32x4{};
    o[dt][1] = f32x4{};
  }
  float m_run[2] = {neg_inf(), neg_inf()};
  f32x4 l_acc[2] = {f32x4{}, f32x4{}};
  const float c = a.scale * kLog2e;

  // kernel arguments the tile loop needs, read once
  const int Nk = a.Nk, Nd = a.Nd;
  const float comp_bias = a.comp_bias;
  int key0 = d128_key0(it, 0);
  int klim = it.cnt > 0 ? Nk : Nd;
  if (it.ntot > 0) {
    d128_issue_k<CT>(it, key0, klim, it.cnt == 0, lk, L, kstride, wave);
    drain_then_barrier();
  }
  for (int t = 0; t < it.ntot; ++t) {
    const bool next = t + 1 < it.ntot;
    const bool comp = t >= it.cnt;
    const bool comp_next = t + 1 >= it.cnt;
    const int key0_next = d128_key0(it, t + 1);
    const int klim_next = comp_next ? Nd : Nk;
    const __amdgpu_buffer_rsrc_t vrs =
        make_rsrc((comp ? it.vdbase : it.vbase) + (int64_t)key0 * vstride, (uint32_t)(klim - key0) * vstride);
    // after the last tile the K copies read nothing (a 0-byte buffer: zeros, no memory
    // access), so that every tile issues the same copies and waits
    const __amdgpu_buffer_rsrc_t krs = make_rsrc((comp_next ? it.kdbase : it.kbase) + (int64_t)key0_next * kstride,
                                                 next ? (uint32_t)(klim_next - key0_next) * kstride : 0u);
    d128_tile<CT>(lk, lv, L, qf, key0, klim, t < it.cnt ? 0.f : comp_bias, c, g, o, m_run, l_acc,
                  [&](int j) { d128_copy_one(lv, vrs, vstride, L.v_off, wave, j); },
                  [&](int j) { d128_copy_one(lk, krs, kstride, L.k_off, wave, j); });
    key0 = key0_next;
    klim = klim_next;
  }

  // O through this wave's 8 KB of the K buffer: every wave has passed the last barrier, so
  // no wave still reads K and no copy into it is in flight.
  d128_store_o_staged<CT>(a, it, o, m_run, l_acc, lk, wave, lane);
}

// fp32 operands: every value is split as x = hi + lo with hi = bf16(x) and
// lo = bf16(x - hi); each product is formed as hi*hi + hi*lo + lo*hi on the bf16 matrix
// cores (about 16 mantissa bits), for QK^T and for PV (P split the same way).  Same
// tiling as block_sparse_fwd_kernel; the hi and lo tiles of K and V^T double the LDS.
__device__ __forceinline__ void split_pair(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  const float h0 = (float)(__bf16)x0, h1 = (float)(__bf16)x1;
  hi = pack2<kBF16>(h0, h1);
  lo = pack2<kBF16>(x0 - h0, x1 - h1);
}

__device__ __forceinline__ void split8(const float* p, u32x4& hi, u32x4& lo) {
  const f32x4 a = reinterpret_cast<const f32x4*>(p)[0];
  const f32x4 b = reinterpret_cast<const f32x4*>(p)[1];
  uint32_t h[4], l[4];
  split_pair(a[0], a[1], h[0], l[0]);
  split_pair(a[2], a[3], h[1], l[1]);
  split_pair(b[0], b[1], h[2], l[2]);
  split_pair(b[2], b[3], h[3], l[3]);
  hi = u32x4{h[0], h[1], h[2], h[3]};
  lo = u32x4{l[0], l[1], l[2], l[3]};
}

template <int D>
__global__ __launch_bounds__(256) void block_sparse_fwd_f32_kernel(FwdArgs a) {
  constexpr int KC = D / 8, DS = D / 16, DT = D / 32;
  __shared__ u32x4 kh[128 * KC], kl[128 * KC];
  __shared__ u32x4 vh[D * 16], vl[D * 16];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int hl = lane >> 5, l32 = lane & 31;
  const int item = a.order ? a.order[blockIdx.x] : (int)blockIdx.x;
  if (item < 0) return;
  const int bh = item / a.nqb;
  const int qb = item - bh * a.nqb;
  const int b = bh / a.H, h = bh - b * a.H;
  const int cnt = a.counts[item];
  const int32_t* list = a.idx + (int64_t)item * a.nkb;
  const float* qbase = (const float*)a.q + ((int64_t)b * a.qs[0] + (int64_t)h * a.qs[1]);
  const float* kbase = (const float*)a.k + ((int64_t)b * a.ks[0] + (int64_t)h * a.ks[1]);
  const float* vbase = (const float*)a.v + ((int64_t)b * a.vs[0] + (int64_t)h * a.vs[1]);

  const int qrow = qb * 128 + wave * 32 + l32;
  u32x4 qh[DS], ql[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s) {
    qh[s] = u32x4{0, 0, 0, 0};
    ql[s] = u32x4{0, 0, 0, 0};
    if (qrow < a.Nq) split8(qbase + (int64_t)qrow * a.qs[2] + s * 16 + hl * 8, qh[s], ql[s]);
  }
  f32x16 o[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) o[i] = f32x16{};
  float m_run = neg_inf(), l_run = 0.f;
  const float c = a.scale * kLog2e;
  const int prow = k_row_perm(l32);
  const int fk = k_swz_kc<KC>(prow);

  for (int it = 0; it < cnt; ++it) {
    const int key0 = list[it] * 128;
    __syncthreads();
#pragma unroll
    for (int c8 = 0; c8 < D / 16; ++c8) {
      const int id = c8 * 256 + tid;
      const int row = id / KC, ch = id % KC;
      const int key = key0 + row;
      u32x4 hi = u32x4{0, 0, 0, 0}, lo = u32x4{0, 0, 0, 0};
      if (key < a.Nk) split8(kbase + (int64_t)key * a.ks[2] + ch * 8, hi, lo);
      kh[row * KC + (ch ^ k_swz_kc<KC>(row))] = hi;
      kl[row * KC + (ch ^ k_swz_kc<KC>(row))] = lo;
    }
#pragma unroll
    for (int i = 0; i < D / 32; ++i) {
      const int id = i * 256 + tid;
      const int dp = id % (D / 2), kg = id / (D / 2);
      uint32_t wh[8], wl[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = key0 + kg * 8 + e;
        f32x2 x = f32x2{0.f, 0.f};
        if (key < a.Nk) x = *reinterpret_cast<const f32x2*>(vbase + (int64_t)key * a.vs[2] + 2 * dp);
        split_pair(x[0], x[1], wh[e], wl[e]);
      }
      u32x4 eh, oh, el, ol;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        eh[j] = (wh[2 * j] & 0xffffu) | (wh[2 * j + 1] << 16);
        oh[j] = (wh[2 * j] >> 16) | (wh[2 * j + 1] & 0xffff0000u);
        el[j] = (wl[2 * j] & 0xffffu) | (wl[2 * j + 1] << 16);
        ol[j] = (wl[2 * j] >> 16) | (wl[2 * j + 1] & 0xffff0000u);
      }
      const int d0 = 2 * dp;
      vh[d0 * 16 + (kg ^ v_swz(d0))] = eh;
      vh[(d0 + 1) * 16 + (kg ^ v_swz(d0 + 1))] = oh;
      vl[d0 * 16 + (kg ^ v_swz(d0))] = el;
      vl[(d0 + 1) * 16 + (kg ^ v_swz(d0 + 1))] = ol;
    }
    __syncthreads();

    f32x16 s[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) s[t] = f32x16{};
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int idx = (t * 32 + prow) * KC + ((2 * ds + hl) ^ fk);
        const u32x4 ah = kh[idx], al = kl[idx];
        s[t] = mfma32x32x16<kBF16>(ah, qh[ds], s[t]);
        s[t] = mfma32x32x16<kBF16>(ah, ql[ds], s[t]);
        s[t] = mfma32x32x16<kBF16>(al, qh[ds], s[t]);
      }
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
    mx = max_xor32(mx);
    const float m_new = fmaxf(m_run, mx * c);
    const float alpha = fast_exp2(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int i = 0; i < DT; ++i) o[i] *= alpha;
    u32x4 ph[4][2], pl[4][2];
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
          uint32_t hv, lv;
          split_pair(v0, v1, hv, lv);
          ph[t][u][e] = hv;
          pl[t][u][e] = lv;
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
          const int idx = R * 16 + ((4 * t + 2 * u + hl) ^ fv);
          const u32x4 ah = vh[idx], al = vl[idx];
          o[dt] = mfma32x32x16<kBF16>(ah, ph[t][u], o[dt]);
          o[dt] = mfma32x32x16<kBF16>(ah, pl[t][u], o[dt]);
          o[dt] = mfma32x32x16<kBF16>(al, ph[t][u], o[dt]);
        }
    }
  }

  const float l = sum_xor32(l_run);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  if (qrow < a.Nq) {
    float* obase = (float*)a.out + ((int64_t)b * a.os[0] + (int64_t)h * a.os[1] + (int64_t)qrow * a.os[2]);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = dt * 32 + 8 * g + 4 * hl;
        store4<kF32>(obase + d, o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv,
                     o[dt][4 * g + 3] * inv);
      }
    if (a.lse != nullptr && hl == 0)
      a.lse[((int64_t)b * a.H + h) * a.Nq + qrow] = cnt > 0 ? (m_run + __log2f(l)) * kLn2 : pos_inf();
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

// Launch order.  Work-group i of the forward runs on XCD i % 8, so the order array decides
// which q-blocks share an XCD's L2 (4 MB).  The q-blocks of one head read the same K/V,
// so the resident work-groups of an XCD (32 CUs x 2) should come from one head at a
// time.  Each head is cut into chunks of about kChunkQb q-blocks (qb = j mod C, C =
// chunks per head).  When the chunk count is not a multiple of 8, the heads of the last,
// partial round are cut finer (C * F chunks each, F = 8 / gcd(their chunks, 8)), so that
// every XCD can get the same share of them.  Whole chunks, then the fine chunks, are dealt
// to the 8 XCDs longest-processing-time first (cost = listed tiles + kQblockCost per q-block), each
// kind at most ceil(count / 8) per XCD, so every XCD gets nearly the same work whatever the
// per-head densities; an XCD runs its whole chunks, then its fine chunks, each kind in
// (head, j) order, and a chunk's q-blocks longest first.  Slots past the end of a shorter
// chunk hold -1.
// Fixed cost of a q-block in the launch-order model, in tiles: a work-group's start (order
// entry, count and list reads), its first K/V copies and its O stores take about as long as
// two tiles (per work-group timestamps at the Z-Image layer: 7.3 us per q-block + 3.45 us
// per tile).
constexpr int kQblockCost = 2;
constexpr int kChunkQb = 128;
constexpr int kMaxChunks = 4096;
constexpr int kMaxOutliers = 1024;
constexpr int kPlanLdsRows = 16384;

__host__ __device__ inline int chunks_per_head(int nqb) {
  const int c = nqb / kChunkQb;
  return c < 1 ? 1 : c;
}

// Chunk layout of a plan: heads [0, nbh_w) in Cw chunks of at most Sw q-blocks, heads
// [nbh_w, nbh) in Cs = Cw * F chunks of at most Ss q-blocks.
struct ChunkLayout {
  int nbh, nbh_w, Cw, Sw, Cs, Ss, nw, ns, cap_w, cap_s;
  __host__ __device__ int slots_per_xcd() const { return cap_w * Sw + cap_s * Ss; }
};

__host__ __device__ inline int gcd_int(int x, int y) {
  while (y != 0) {
    const int t = x % y;
    x = y;
    y = t;
  }
  return x;
}

__host__ __device__ inline ChunkLayout chunk_layout(int nbh, int nqb) {
  ChunkLayout L;
  L.nbh = nbh;
  L.Cw = chunks_per_head(nqb);
  L.Sw = (nqb + L.Cw - 1) / L.Cw;
  const int rem = (nbh * L.Cw) % kXcds;  // chunks of the partial last round
  const int nsplit = rem == 0 ? 0 : (rem + L.Cw - 1) / L.Cw;
  L.nbh_w = nbh - nsplit;
  int F = kXcds / gcd_int(nsplit * L.Cw, kXcds);
  while (F > 1 && L.Cw * F > nqb) F >>= 1;  // a fine chunk keeps at least one q-block
  L.Cs = L.Cw * F;
  L.Ss = (nqb + L.Cs - 1) / L.Cs;
  L.nw = L.nbh_w * L.Cw;
  L.ns = nsplit * L.Cs;
  L.cap_w = (L.nw + kXcds - 1) / kXcds;
  L.cap_s = (L.ns + kXcds - 1) / kXcds;
  return L;
}

constexpr int kPlanThreads = 1024;
constexpr int kPlanWaves = kPlanThreads / 64;

// Chunked plans keep a chunk table after the launch slots of the order buffer, written by
// plan_order_kernel and read by plan_chunk_sort_kernel: [0, 8) q-blocks per XCD, [8, 24)
// cost sum per XCD (low, high word), [24] outliers taken out (1) or not (0), then per chunk
// ch [32 + 2ch] its first slot along its XCD's sequence and [33 + 2ch] its XCD.
constexpr int kMetaHead = 32;
// [25] 1 when the launch slots were copied from the launch-order cache (the chunk pass then
// has nothing to do), [26], [27] the hash of the plan's tile counts (low, high word).
constexpr int kMetaCopied = 25, kMetaHashLo = 26, kMetaHashHi = 27;

// Launch-order cache: int32 [kCacheHead + entries * (kCacheEntryHead + S)], S =
// plan_order_slots() of the shape, zero-filled by its owner before first use and used by
// one stream at a time.  Head: [0] the next entry to fill, [1] chunk-pass groups done (the
// last one inserts the finished order and sets it back to zero).  Entry: [0] 1 when filled,
// [1], [2] the hash of its tile counts, then the S ints of its order buffer.  The launch
// order depends only on the shape and the tile counts, so a plan whose counts hash like a
// filled entry's takes that entry's order instead of ranking the chunks again.  A hash
// collision can only cost balance, never correctness: every order of a shape is a
// permutation of the same q-blocks.
constexpr int kCacheHead = 4, kCacheEntryHead = 4;

// SplitMix64's output function (Steele, Lea, Flood 2014): a 64-bit mixer.
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x ^= x >> 30;
  x *= 0xbf58476d1ce4e5b9ull;
  x ^= x >> 27;
  x *= 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off, 64);
    v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}

__host__ __device__ inline int chunk_size(const ChunkLayout& L, int nqb, int ch) {
  const int C = ch < L.nw ? L.Cw : L.Cs;
  const int j = ch < L.nw ? ch % L.Cw : (ch - L.nw) % L.Cs;
  return (nqb - j + C - 1) / C;
}

// chunk ch -> (head, residue j, modulus)
__device__ __forceinline__ void chunk_head(const ChunkLayout& L, int ch, int& bh, int& j, int& C) {
  if (ch < L.nw) {
    bh = ch / L.Cw;
    j = ch - bh * L.Cw;
    C = L.Cw;
  } else {
    const int f = ch - L.nw;
    bh = L.nbh_w + f / L.Cs;
    j = f % L.Cs;
    C = L.Cs;
  }
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <bool STAGED>
__global__ __launch_bounds__(kPlanThreads) void plan_order_kernel(PlanArgs a) {
  __shared__ int cost[kMaxChunks];
  __shared__ int16_t sorted[kMaxChunks + 2 * kXcds];  // later also 8 * (cap_s + cap_w)
  __shared__ int scost[kMaxChunks];                   // cost of the r-th ranked chunk
  __shared__ uint8_t xcd[kMaxChunks];
  __shared__ int16_t pos[kMaxChunks];
  // The passes below read each q-block's tile count several times.  STAGED (rows <=
  // kPlanLdsRows): they are copied to LDS once (eight coalesced loads in flight per
  // thread) and read there; otherwise they are read from global memory.
  __shared__ int cnt_lds[STAGED ? kPlanLdsRows : 1];
  __shared__ unsigned long long xsum[kXcds];
  __shared__ int xcnt[kXcds], nout[kXcds], nlist;
  __shared__ int outl[kMaxOutliers], outl_c[kMaxOutliers];
  __shared__ uint8_t outl_x[kMaxOutliers];
  __shared__ int16_t nonout[kMaxChunks];
  __shared__ unsigned long long hash_part[kPlanWaves];
  __shared__ int hit;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  const ChunkLayout L = chunk_layout(a.rows / a.nqb, a.nqb);
  const int nch = L.nw + L.ns;
  const int total = L.slots_per_xcd() * kXcds;
  const int S = total + kMetaHead + 2 * nch;  // ints of the order buffer
  int32_t* meta = a.order + total;
  if constexpr (STAGED) {
    for (int base = 0; base < a.rows; base += 8 * kPlanThreads) {
      int v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = base + u * kPlanThreads + tid;
        v[u] = i < a.rows ? a.counts[i] : 0;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int i = base + u * kPlanThreads + tid;
        if (i < a.rows) cnt_lds[i] = v[u];
      }
    }
  }
  auto counts = [&](int row) __attribute__((always_inline)) {
    if constexpr (STAGED) return cnt_lds[row];
    else return a.counts[row];
  };
  // With a launch-order cache: the hash of the tile counts (a wrapping sum of one mixed
  // word per row, so any thread may take any row), then the first filled entry with that
  // hash, whose order is copied.
  uint64_t hash = 0;
  if (a.cache != nullptr) {
    __syncthreads();  // counts staged
    uint64_t hs = 0;
    for (int row = tid; row < a.rows; row += kPlanThreads)
      hs += mix64(((uint64_t)(uint32_t)row << 32) | (uint32_t)counts(row));
    hs = wave_sum_u64(hs);
    if (lane == 0) hash_part[wv] = hs;
    __syncthreads();
    hash = mix64(((uint64_t)(uint32_t)a.rows << 32) | (uint32_t)a.nqb);
    for (int w = 0; w < kPlanWaves; ++w) hash += hash_part[w];
    if (wv == 0) {
      int found = -1;
      for (int e0 = 0; e0 < a.cache_entries && found < 0; e0 += 64) {
        const int e = e0 + lane;
        bool m = false;
        if (e < a.cache_entries) {
          const int32_t* eh = a.cache + kCacheHead + (int64_t)e * (kCacheEntryHead + S);
          m = eh[0] == 1 && (uint32_t)eh[1] == (uint32_t)hash && (uint32_t)eh[2] == (uint32_t)(hash >> 32);
        }
        const uint64_t b = __ballot(m);
        if (b != 0) found = e0 + __ffsll((unsigned long long)b) - 1;
      }
      if (lane == 0) hit = found;
    }
    __syncthreads();
    if (hit >= 0) {
      const int32_t* src = a.cache + kCacheHead + (int64_t)hit * (kCacheEntryHead + S) + kCacheEntryHead;
      for (int i = tid; i < S; i += kPlanThreads) a.order[i] = i == total + kMetaCopied ? 1 : src[i];
      return;
    }
  }
  for (int i = tid; i < total; i += kPlanThreads) a.order[i] = -1;
  if (tid < kXcds) {
    xsum[tid] = 0;
    xcnt[tid] = nout[tid] = 0;
  }
  if (tid == 0) nlist = 0;
  __syncthreads();
  // chunk costs: one wave per chunk, its lanes striding over the chunk's q-blocks
  for (int ch = wv; ch < nch; ch += kPlanWaves) {
    int bh, j, C;
    chunk_head(L, ch, bh, j, C);
    int w = 0;
    for (int qb = j + lane * C; qb < a.nqb; qb += 64 * C) w += counts(bh * a.nqb + qb) + kQblockCost;
    w = wave_sum_i32(w);
    if (lane == 0) cost[ch] = w;
  }
  __syncthreads();
  // rank by cost desc, index asc, within each kind (whole chunks, then fine chunks)
  for (int ch = tid; ch < nch; ch += kPlanThreads) {
    const int lo = ch < L.nw ? 0 : L.nw, hi = ch < L.nw ? L.nw : nch;
    const int w = cost[ch];
    int r = lo;
    for (int c2 = lo; c2 < hi; ++c2) r += (cost[c2] > w) || (cost[c2] == w && c2 < ch);
    sorted[r] = (int16_t)ch;
    scost[r] = w;
  }
  __syncthreads();
  // Longest processing time first, one kind after the other: each chunk to the XCD with
  // the least load (the lowest index among equals) that has room for one more of its kind.
  // Wave 0 walks the ranking 64 chunks at a time (lane k holds the k-th chunk's cost).
  // Lane x < 8 holds XCD x's load and count; the choice is the minimum over those lanes of
  // load * 8 + x (three DPP steps), or, when the loads could pass 2^28, a scalar scan.
  if (wv == 0) {
    int64_t all = 0;
    for (int r = lane; r < nch; r += 64) all += scost[r];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) all += __shfl_xor(all, off, 64);
    const bool small = all < (1ll << 28);  // every load * 8 + 7 fits an int
    int load = 0, nx = 0;  // lane x < 8: XCD x
    for (int kind = 0; kind < 2; ++kind) {
      const int lo = kind == 0 ? 0 : L.nw, hi = kind == 0 ? L.nw : nch;
      const int cap = kind == 0 ? L.cap_w : L.cap_s;
      nx = 0;
      for (int rb = lo; rb < hi; rb += 64) {
        const int rr = rb + lane;
        const int wl = rr < hi ? scost[rr] : 0;
        int mine = 0;
        const int m = min(64, hi - rb);
        for (int k = 0; k < m; ++k) {
          const int w = __builtin_amdgcn_readlane(wl, k);
          int best;
          if (small) {
            int key = (lane < kXcds && nx < cap) ? load * 8 + lane : 0x7fffffff;
            key = min(key, __builtin_amdgcn_mov_dpp(key, 0xB1, 0xF, 0xF, false));   // lane ^ 1
            key = min(key, __builtin_amdgcn_mov_dpp(key, 0x4E, 0xF, 0xF, false));   // lane ^ 2
            key = min(key, __builtin_amdgcn_mov_dpp(key, 0x141, 0xF, 0xF, false));  // 7 - lane (within 8)
            best = __builtin_amdgcn_readfirstlane(key) & 7;
          } else {
            best = -1;
            int bl = 0;
#pragma unroll
            for (int x = 0; x < kXcds; ++x) {
              const int lx = __builtin_amdgcn_readlane(load, x), nxx = __builtin_amdgcn_readlane(nx, x);
              const bool take = nxx < cap && (best < 0 || lx < bl);
              best = take ? x : best;
              bl = take ? lx : bl;
            }
          }
          load += lane == best ? w : 0;
          nx += lane == best ? 1 : 0;
          mine = lane == k ? best : mine;
        }
        if (rr < hi) xcd[sorted[rr]] = (uint8_t)mine;
      }
    }
  }
  __syncthreads();
  // each chunk's position among its XCD's chunks of the same kind (chunk order), and the
  // XCD totals
  for (int ch = tid; ch < nch; ch += kPlanThreads) {
    const int lo = ch < L.nw ? 0 : L.nw;
    const int x = xcd[ch];
    int p = 0;
    for (int c2 = lo; c2 < ch; ++c2) p += xcd[c2] == x;
    pos[ch] = (int16_t)p;
    atomicAdd(&xsum[x], (unsigned long long)cost[ch]);
    atomicAdd(&xcnt[x], chunk_size(L, a.nqb, ch));
  }
  // Sequence of each XCD: its outliers first (q-blocks costing more than twice the XCD's
  // mean, longest first: a long row started late ends the launch late), then its fine
  // chunks, then its whole chunks (each kind by position), each chunk's other q-blocks
  // longest first.  Outliers are fewer than half of an XCD's q-blocks; past kMaxOutliers
  // in the whole plan none are taken out (the chunk sequence alone).
  int16_t* seq = sorted;   // the ranking is spent: it becomes each XCD's chunk sequence
  const int per_x = L.cap_s + L.cap_w;
  __syncthreads();
  for (int i = tid; i < per_x * kXcds; i += kPlanThreads) seq[i] = -1;
  __syncthreads();
  for (int ch = tid; ch < nch; ch += kPlanThreads)
    seq[xcd[ch] * per_x + (ch < L.nw ? L.cap_s : 0) + pos[ch]] = (int16_t)ch;
  // outliers, one wave per chunk: a q-block of `c` tiles on XCD x is an outlier when
  // (c + kQblockCost) * count > 2 * sum; nonout[ch] holds the chunk's outlier count for now
  for (int ch = wv; ch < nch; ch += kPlanWaves) {
    int bh, j, C;
    chunk_head(L, ch, bh, j, C);
    const int x = xcd[ch];
    const int64_t xc = xcnt[x], xs2 = 2 * (int64_t)xsum[x];
    int nch_out = 0;
    for (int q0 = j; q0 < a.nqb; q0 += 64 * C) {
      const int qb = q0 + lane * C;
      const int row = bh * a.nqb + qb;
      const bool is_out = qb < a.nqb && (int64_t)(counts(row) + kQblockCost) * xc > xs2;
      const uint64_t mk = __ballot(is_out);
      const int n_here = __popcll(mk);
      if (n_here == 0) continue;
      int base = 0;
      if (lane == 0) base = atomicAdd(&nlist, n_here);
      base = __shfl(base, 0, 64);
      const int k = base + __popcll(mk & ((1ull << lane) - 1ull));
      if (is_out && k < kMaxOutliers) outl[k] = row;
      nch_out += n_here;
    }
    if (lane == 0) {
      nonout[ch] = (int16_t)nch_out;
      if (nch_out) atomicAdd(&nout[x], nch_out);
    }
  }
  __syncthreads();
  const bool use_out = nlist <= kMaxOutliers;
  for (int ch = tid; ch < nch; ch += kPlanThreads) {  // non-outlier count per chunk
    const int S = chunk_size(L, a.nqb, ch);
    nonout[ch] = (int16_t)(use_out ? S - nonout[ch] : S);
  }
  if (use_out) {  // XCD and tile count of every listed outlier
    for (int k = tid; k < nlist; k += kPlanThreads) {
      const int r = outl[k];
      const int bh = r / a.nqb, qb = r - bh * a.nqb;
      const bool fine = bh >= L.nbh_w;
      const int C = fine ? L.Cs : L.Cw;
      const int ch = fine ? L.nw + (bh - L.nbh_w) * L.Cs + qb % C : bh * L.Cw + qb % C;
      outl_x[k] = xcd[ch];
      outl_c[k] = counts(r);
    }
  }
  __syncthreads();
  if (tid < kXcds) {  // offsets along each XCD's chunk sequence
    const int x = tid;
    int off = use_out ? nout[x] : 0;
    for (int k = 0; k < per_x; ++k) {
      const int ch = seq[x * per_x + k];
      if (ch < 0) continue;
      meta[kMetaHead + 2 * ch] = off;
      off += nonout[ch];
    }
    meta[x] = xcnt[x];
    meta[8 + 2 * x] = (int32_t)(xsum[x] & 0xffffffffull);
    meta[9 + 2 * x] = (int32_t)(xsum[x] >> 32);
  }
  if (tid == 0) {
    meta[24] = use_out ? 1 : 0;
    meta[kMetaCopied] = 0;
    meta[kMetaHashLo] = (int32_t)(uint32_t)hash;
    meta[kMetaHashHi] = (int32_t)(uint32_t)(hash >> 32);
  }
  for (int ch = tid; ch < nch; ch += kPlanThreads) meta[kMetaHead + 2 * ch + 1] = xcd[ch];
  // Outliers: rank among the XCD's outliers by cost desc, then row asc.
  if (use_out) {
    for (int k = tid; k < nlist; k += kPlanThreads) {
      const int r = outl[k], x = outl_x[k], c = outl_c[k];
      int slot = 0;
      for (int k2 = 0; k2 < nlist; ++k2) {
        const int c2 = outl_c[k2];
        slot += (k2 != k) & (outl_x[k2] == x) & ((c2 > c) | ((c2 == c) & (outl[k2] < r)));
      }
      a.order[slot * kXcds + x] = r;
    }
  }
}

// The other q-blocks of chunk blockIdx.x (one wave; the chunk table from plan_order_kernel).
// A chunk has at most 255 q-blocks (chunks split heads of >= 128 q-blocks into pieces of
// 128-255), four per lane.  Their keys go to LDS in q order: count * 256 + (255 - k) for
// the k-th q-block of the chunk (more tiles first, then lower q), -1 for an outlier and
// past the chunk's end.  Every lane ranks its four against the row, 16 bytes per broadcast
// read, with one comparison per pair and no branches.
__global__ __launch_bounds__(64) void plan_chunk_sort_kernel(PlanArgs a) {
  __shared__ int keys[256];
  const int lane = (int)threadIdx.x;
  const int ch = (int)blockIdx.x;
  const ChunkLayout L = chunk_layout(a.rows / a.nqb, a.nqb);
  const int total = L.slots_per_xcd() * kXcds;
  const int32_t* meta = a.order + total;
  if (a.cache != nullptr && meta[kMetaCopied] == 1) return;  // slots copied from the cache
  int bh, j, C;
  chunk_head(L, ch, bh, j, C);
  const int S = (a.nqb - j + C - 1) / C;
  const int off = meta[kMetaHead + 2 * ch], x = meta[kMetaHead + 2 * ch + 1];
  const bool use_out = meta[24] != 0;
  const int64_t xsum = (int64_t)(((uint64_t)(uint32_t)meta[9 + 2 * x] << 32) | (uint32_t)meta[8 + 2 * x]);
  const int64_t xc = use_out ? meta[x] : 0, xs2 = 2 * xsum;
  int key[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int k = lane + 64 * u;
    key[u] = -1;
    if (k < S) {
      const int c = a.counts[bh * a.nqb + j + k * C];
      if ((int64_t)(c + kQblockCost) * xc <= xs2) key[u] = c * 256 + (255 - k);
    }
    keys[k] = key[u];
  }
  __syncthreads();
  int rank[4] = {0, 0, 0, 0};
  for (int k2 = 0; k2 < S; k2 += 4) {
    const i32x4 v = *reinterpret_cast<const i32x4*>(keys + k2);
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int u = 0; u < 4; ++u) rank[u] += v[e] > key[u];
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int k = lane + 64 * u;
    if (key[u] >= 0) a.order[(off + rank[u]) * kXcds + x] = bh * a.nqb + j + k * C;
  }
  if (a.cache == nullptr) return;
  // The last group to finish copies the whole order buffer into the cache entry to fill next
  // (device-scope fences around the completion count; the other groups' slots are read with
  // agent-scope loads).
  __threadfence();
  int last = 0;
  if (lane == 0) last = atomicAdd(a.cache + 1, 1) == (int)gridDim.x - 1;
  last = __shfl(last, 0, 64);
  if (!last) return;
  __threadfence();
  const int ints = total + kMetaHead + 2 * (L.nw + L.ns);  // of the order buffer
  const int e = __hip_atomic_load(a.cache, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) % a.cache_entries;
  int32_t* ent = a.cache + kCacheHead + (int64_t)e * (kCacheEntryHead + ints);
  for (int i = lane; i < ints; i += 64)
    ent[kCacheEntryHead + i] = __hip_atomic_load(a.order + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (lane == 0) {
    ent[0] = 1;
    ent[1] = meta[kMetaHashLo];
    ent[2] = meta[kMetaHashHi];
    a.cache[0] = (e + 1) % a.cache_entries;
    a.cache[1] = 0;
  }
}

// Fallback when a plan has more chunks than the ordering kernel holds: XCD x gets the
// q-blocks qb = x (mod 8) of every head, head by head, longest first within a head.
__global__ __launch_bounds__(256) void plan_order_interleaved_kernel(PlanArgs a) {
  const int slices = (a.nqb + kXcds - 1) / kXcds;
  const int total = a.rows / a.nqb * slices * kXcds;
  for (int i = threadIdx.x; i < total; i += blockDim.x) a.order[i] = -1;
  __syncthreads();
  for (int row = threadIdx.x; row < a.rows; row += blockDim.x) {
    const int bh = row / a.nqb, qb = row - bh * a.nqb;
    const int x = qb % kXcds;
    const int c = a.counts[row];
    int rank = 0;
    for (int q2 = x; q2 < a.nqb; q2 += kXcds) {
      const int c2 = a.counts[bh * a.nqb + q2];
      rank += (c2 > c) || (c2 == c && q2 < qb);
    }
    a.order[(bh * slices + rank) * kXcds + x] = row;
  }
}

static bool chunked_order(int rows, int nqb) {
  const ChunkLayout L = chunk_layout(rows / nqb, nqb);
  return L.nw + L.ns <= kMaxChunks;
}

// Work-groups of a forward launch over a plan's order: its launch slots.
static int plan_launch_slots(int rows, int nqb) {
  if (rows == 0 || nqb == 0) return 0;
  const int nbh = rows / nqb;
  if (!chunked_order(rows, nqb)) return nbh * ((nqb + kXcds - 1) / kXcds) * kXcds;
  return chunk_layout(nbh, nqb).slots_per_xcd() * kXcds;
}

// int32 entries of the order buffer: the launch slots, then (chunked plans) the chunk table.
int plan_order_slots(int rows, int nqb) {
  const int slots = plan_launch_slots(rows, nqb);
  if (slots == 0 || !chunked_order(rows, nqb)) return slots;
  const ChunkLayout L = chunk_layout(rows / nqb, nqb);
  return slots + kMetaHead + 2 * (L.nw + L.ns);
}

int64_t plan_order_cache_ints(int rows, int nqb, int entries) {
  return kCacheHead + (int64_t)entries * (kCacheEntryHead + plan_order_slots(rows, nqb));
}

hipError_t launch_block_sparse_plan(const PlanArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  plan_rows_kernel<<<(a.rows + 3) / 4, 256, 0, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.order == nullptr) return e;
  if (chunked_order(a.rows, a.nqb)) {
    if (a.rows <= kPlanLdsRows)
      plan_order_kernel<true><<<1, kPlanThreads, 0, stream>>>(a);
    else
      plan_order_kernel<false><<<1, kPlanThreads, 0, stream>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const ChunkLayout L = chunk_layout(a.rows / a.nqb, a.nqb);
    plan_chunk_sort_kernel<<<L.nw + L.ns, 64, 0, stream>>>(a);
  } else
    plan_order_interleaved_kernel<<<1, 256, 0, stream>>>(a);
  return hipGetLastError();
}

static int fwd_grid(const FwdArgs& a) {
  const int rows = a.B * a.H * a.nqb;
  return a.order ? plan_launch_slots(rows, a.nqb) : rows;
}

template <int IT, int CT>
static hipError_t launch_fwd_dt(const FwdArgs& a, int D, hipStream_t stream) {
  const int grid = fwd_grid(a);
  if (D == 128)
    block_sparse_fwd_d128_kernel<CT><<<grid, 256, 0, stream>>>(a);
  else if (D == 64)
    block_sparse_fwd_kernel<IT, CT, 64><<<grid, 256, 0, stream>>>(a);
  else
    block_sparse_fwd_kernel<IT, CT, 32><<<grid, 256, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_block_sparse_fwd(const FwdArgs& a, int dtype, int D, hipStream_t stream) {
  if (a.B * a.H * a.nqb == 0) return hipSuccess;
  switch (dtype) {
    case kBF16: return launch_fwd_dt<kBF16, kBF16>(a, D, stream);
    case kF16: return launch_fwd_dt<kF16, kF16>(a, D, stream);
    default: {
      const int grid = fwd_grid(a);
      if (D == 128)
        block_sparse_fwd_f32_kernel<128><<<grid, 256, 0, stream>>>(a);
      else if (D == 64)
        block_sparse_fwd_f32_kernel<64><<<grid, 256, 0, stream>>>(a);
      else
        block_sparse_fwd_f32_kernel<32><<<grid, 256, 0, stream>>>(a);
      return hipGetLastError();
    }
  }
}

}  // namespace sa
