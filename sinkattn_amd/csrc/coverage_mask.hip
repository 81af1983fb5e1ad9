// Direct-mean coverage mask for gfx950, bit-exact with the reference's CPU torch path.
//
// Reference: `_build_direct_mean_coverage_mask` and `_build_offline_required_mask`
// (sinkattention/sparse_attention.py:241-376).  The reference runs on CPU tensors, so
// the bits of its mask are fixed by CPU torch's arithmetic, which this kernel restates:
//   * row sums (`x.sum(-1)`) follow ATen's vectorised inner reduction: 8-lane fp32
//     vectors, 4 interleaved vector accumulators with ATen's multi-level cascade, the
//     accumulators folded 0+1+2+3, then the scalar tail summed from 0 and the 8 lanes
//     added in lane order (all fp32);
//   * `torch.cumsum` on fp32 accumulates in fp64 and rounds every prefix to fp32;
//   * `coverage * total` is one fp32 multiply; comparisons with 1e-6 are fp32;
//   * `torch.sort(descending=True)` is libstdc++ `std::sort` on (value, index) pairs with
//     comparator `(isnan(a) && !isnan(b)) || a > b` (unstable).
// One 64-thread work-group handles one (head, query-block) row.  The row sums run ATen's
// 32 accumulator chains one per lane; the row is sorted with a register-resident bitonic
// network keyed (value desc, index asc).  Values, prefix sums and the cut k
// do not depend on how ties are ordered; the selected set does only when a tie group
// straddles the cut (v[k-1] == v[k]) or the empty-row fallback picks among tied maxima.
// Those rows are re-sorted with a single-lane emulation of libstdc++'s introsort so the
// permutation matches the reference exactly.  Rows shorter than 8 elements take ATen's
// scalar inner sum (same accumulator scheme on scalars).  A second pass applies the
// reference's global empty-row fallback and writes the per-row index lists.

#include "common.h"
#include "kernels.h"

// Every product and sum here must round exactly like the reference's CPU arithmetic:
// no fused multiply-adds (e.g. coverage * total - selected must round the product).
#pragma clang fp contract(off)

namespace sa {

// Row capacity: instances hold rows of 256 * C key blocks for C = 1, 2, 4, 8, 16 (5.3 KB
// to 84 KB of LDS), so short rows keep many work-groups resident per CU.
constexpr int kMaskMaxN = 4096;
// Rows per work-group of the fixup pass.
constexpr int kFixupRows = 16;

// --- ATen-compatible fp32 row sum ---------------------------------------------------
// x[i] * mul(i) is summed; mul is 1 (plain) or the 0/1 required flag (masked sum).
struct RowView {
  const float* x;
  int n;
  int qb, req_q, req_k;
  bool masked;
  __device__ __forceinline__ float at(int i) const {
    if (!masked) return x[i];
    const bool req = (qb < req_q) || (i < req_k);
    return x[i] * (req ? 1.f : 0.f);
  }
};

__device__ __forceinline__ int ceil_log2(int64_t v) {
  if (v <= 1) return 0;
  return 64 - __clzll((unsigned long long)(v - 1));
}

// ATen's row_sum over `nunits` units of L lanes (L = 8: fp32 vectors, L = 1: scalars):
// 4 interleaved accumulators with a 4-level cascade, leftover units into accumulator 0,
// accumulators folded 0+1+2+3.  Element (unit u, lane e) is r.at(u * L + e).
template <int L>
__device__ void aten_units_sum(const RowView& r, int nunits, float* out) {
  float acc[4][4][L];
#pragma unroll
  for (int l = 0; l < 4; ++l)
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int e = 0; e < L; ++e) acc[l][k][e] = 0.f;
  const int size_ilp = nunits / 4;
  const int level_power = max(4, ceil_log2(size_ilp) / 4);
  const int level_step = 1 << level_power;
  const int level_mask = level_step - 1;
  int i = 0;
  while (i + level_step <= size_ilp) {
    for (int j = 0; j < level_step; ++j, ++i) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < L; ++e) acc[0][k][e] += r.at((i * 4 + k) * L + e);
    }
#pragma unroll
    for (int j = 1; j < 4; ++j) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < L; ++e) {
          acc[j][k][e] += acc[j - 1][k][e];
          acc[j - 1][k][e] = 0.f;
        }
      const int mask = level_mask << (j * level_power);
      if ((i & mask) != 0) break;
    }
  }
  for (; i < size_ilp; ++i) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int e = 0; e < L; ++e) acc[0][k][e] += r.at((i * 4 + k) * L + e);
  }
#pragma unroll
  for (int j = 1; j < 4; ++j)
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int e = 0; e < L; ++e) acc[0][k][e] += acc[j][k][e];
  for (int v = size_ilp * 4; v < nunits; ++v)
#pragma unroll
    for (int e = 0; e < L; ++e) acc[0][0][e] += r.at(v * L + e);
#pragma unroll
  for (int k = 1; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < L; ++e) acc[0][0][e] += acc[0][k][e];
#pragma unroll
  for (int e = 0; e < L; ++e) out[e] = acc[0][0][e];
}

// Contiguous fp32 row sum in ATen's order: rows of >= 8 elements take the vectorised
// inner sum (8-lane units, then the scalar tail summed from 0 and the lanes added in
// order); shorter rows take the scalar inner sum (the same scheme on scalars).
__device__ float aten_row_sum(const RowView& r) {
  const int n = r.n;
  if (n < 8) {
    float one[1];
    aten_units_sum<1>(r, n, one);
    return one[0];
  }
  const int vec_size = n / 8;
  float lanes[8];
  aten_units_sum<8>(r, vec_size, lanes);
  float fin = 0.f;
  for (int t = vec_size * 8; t < n; ++t) fin += r.at(t);
#pragma unroll
  for (int e = 0; e < 8; ++e) fin += lanes[e];
  return fin;
}

// --- libstdc++ std::sort emulation on (value, index) pairs, descending comparator -----
// An entry packs the value's bits (low word) and its index (high word), so a move is one
// 64-bit LDS access.  `e` points one entry into an array of n + 2 entries: the scans read
// one entry ahead (e[-1] .. e[n]), always inside the array, and a value read ahead is
// only compared once the original algorithm reaches its position.
__device__ __forceinline__ float pval(uint64_t x) { return __uint_as_float((uint32_t)x); }
__device__ __forceinline__ int pidx(uint64_t x) { return (int)(x >> 32); }
__device__ __forceinline__ uint64_t pmake(float v, int i) {
  return ((uint64_t)(uint32_t)i << 32) | __float_as_uint(v);
}
// The comparator: x goes before y.
__device__ __forceinline__ bool pcomp(float x, float y) {
  return (__builtin_isnan(x) && !__builtin_isnan(y)) || (x > y);
}

__device__ void std_move_median_to_first(uint64_t* e, int result, int a, int b, int c) {
  const uint64_t ea = e[a], eb = e[b], ec = e[c];
  const float va = pval(ea), vb = pval(eb), vc = pval(ec);
  int pick;
  uint64_t ep;
  if (pcomp(va, vb)) {
    if (pcomp(vb, vc)) { pick = b; ep = eb; }
    else if (pcomp(va, vc)) { pick = c; ep = ec; }
    else { pick = a; ep = ea; }
  } else if (pcomp(va, vc)) {
    pick = a; ep = ea;
  } else if (pcomp(vb, vc)) {
    pick = c; ep = ec;
  } else {
    pick = b; ep = eb;
  }
  const uint64_t er = e[result];
  e[result] = ep;
  e[pick] = er;
}

// __adjust_heap(first, hole, len, value) on [base, base+len)
__device__ void std_adjust_heap(uint64_t* e, int base, int hole, int len, uint64_t val) {
  const int top = hole;
  int second = hole;
  while (second < (len - 1) / 2) {
    second = 2 * (second + 1);
    if (pcomp(pval(e[base + second]), pval(e[base + second - 1]))) second--;
    e[base + hole] = e[base + second];
    hole = second;
  }
  if ((len & 1) == 0 && second == (len - 2) / 2) {
    second = 2 * (second + 1);
    e[base + hole] = e[base + second - 1];
    hole = second - 1;
  }
  // __push_heap
  const float vv = pval(val);
  int parent = (hole - 1) / 2;
  while (hole > top && pcomp(pval(e[base + parent]), vv)) {
    e[base + hole] = e[base + parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  e[base + hole] = val;
}

__device__ void std_heap_sort(uint64_t* e, int first, int last) {
  const int len = last - first;
  if (len >= 2) {  // __make_heap
    int parent = (len - 2) / 2;
    while (true) {
      std_adjust_heap(e, first, parent, len, e[first + parent]);
      if (parent == 0) break;
      parent--;
    }
  }
  // __sort_heap
  while (last - first > 1) {
    --last;
    const uint64_t val = e[last];
    e[last] = e[first];
    std_adjust_heap(e, first, 0, last - first, val);
  }
}

__device__ void std_unguarded_linear_insert(uint64_t* e, int last) {
  const uint64_t val = e[last];
  const float vv = pval(val);
  int next = last - 1;
  uint64_t en = e[next], en1 = e[next - 1];
  while (pcomp(vv, pval(en))) {
    e[last] = en;
    last = next;
    --next;
    en = en1;
    en1 = e[next - 1];
  }
  e[last] = val;
}

__device__ void std_insertion_sort(uint64_t* e, int first, int last) {
  if (first == last) return;
  for (int i = first + 1; i != last; ++i) {
    const uint64_t ei = e[i];
    if (pcomp(pval(ei), pval(e[first]))) {
      for (int j = i; j > first; --j) e[j] = e[j - 1];
      e[first] = ei;
    } else {
      std_unguarded_linear_insert(e, i);
    }
  }
}

// __unguarded_partition(e + first, e + last, e + pivot) computed by the whole wave, with
// the serial scans' result.  Call a position an L-stop when its original value is not
// before the pivot and an R-stop when it is not after it.  The k-th iteration of the
// serial loop stops its left scan at the k-th L-stop l_k and its right scan at the k-th
// R-stop from the right r_k, and swaps them while l_k < r_k: until the scans cross they
// read only untouched positions.  With s such swaps, the next left scan stops at l_s or,
// failing an untouched L-stop before it, at r_{s-1} (which now holds an L-stop's value):
// the cut is min(l_s, r_{s-1}).  The 2s swapped positions are distinct.  `lp` and `rp`
// receive the stop positions (last - first entries each).  All 64 lanes call it.
__device__ int wave_unguarded_partition(uint64_t* e, int first, int last, int pivot, int* lp,
                                        int* rp, int lane) {
  const float pv = pval(e[pivot]);
  const uint64_t below = (1ull << lane) - 1ull;
  int nl = 0, nr = 0;
  for (int c0 = first; c0 < last; c0 += 64) {
    const int i = c0 + lane;       // ascending positions
    const int j = last - 1 - (c0 - first) - lane;  // descending positions
    const bool ini = i < last, inj = j >= first;
    const float xi = ini ? pval(e[i]) : 0.f;
    const float xj = inj ? pval(e[j]) : 0.f;
    const bool isl = ini && !pcomp(xi, pv);
    const bool isr = inj && !pcomp(pv, xj);
    const uint64_t bl = __ballot(isl), br = __ballot(isr);
    if (isl) lp[nl + __popcll(bl & below)] = i;
    if (isr) rp[nr + __popcll(br & below)] = j;
    nl += __popcll(bl);
    nr += __popcll(br);
  }
  __syncthreads();
  // l_k < r_k holds for a prefix of k; count it.
  int sw = 0;
  const int kmax = min(nl, nr);
  for (int k0 = 0; k0 < kmax; k0 += 64) {
    const int k = k0 + lane;
    sw += __popcll(__ballot(k < kmax && lp[k] < rp[k]));
  }
  int cut = sw < nl ? lp[sw] : 0x7fffffff;
  if (sw > 0) cut = min(cut, rp[sw - 1]);
  for (int k0 = 0; k0 < sw; k0 += 64) {
    const int k = k0 + lane;
    if (k < sw) {
      const int a = lp[k], b = rp[k];
      const uint64_t ea = e[a], eb = e[b];
      e[a] = eb;
      e[b] = ea;
    }
  }
  __syncthreads();
  return cut;
}

// libstdc++'s std::sort(e, e + n) as far as positions [p0, p1) are concerned: after the
// call those positions hold exactly what the full sort puts there.  Introsort's
// sub-ranges are sorted independently of each other, and its final insertion pass never
// moves an element across the boundary of a sub-range left by the partitions (the
// elements before a boundary are never strictly after those behind it), so it acts as an
// insertion sort of each such range.  The walk therefore follows only partitions whose
// range meets [p0, p1) and insertion-sorts only the leftover ranges it reaches; with
// [0, n) it is the full sort.  `stk` is a 3 x 64-entry LDS stack of pending ranges (at
// most 2*log2(n) + 1 at once).
// Partitions are done by the whole wave; median selection, heap sort and the leftover
// insertion sorts stay on lane 0.  `lp` and `rp` hold n entries each.  All 64 lanes call it.
__device__ void wave_sort_positions(uint64_t* e, int n, int p0, int p1, int* stk, int* lp,
                                    int* rp, int lane) {
  if (n <= 1 || p0 >= p1) return;
  constexpr int kThreshold = 16;
  // The stack is written by every lane with the same values and read by all of them.
  int* st_first = stk;
  int* st_last = stk + 64;
  int* st_depth = stk + 128;
  int sp = 0;
  st_first[sp] = 0; st_last[sp] = n; st_depth[sp] = 2 * (31 - __clz(n)); ++sp;
  while (sp > 0) {
    --sp;
    int first = st_first[sp], last = st_last[sp], depth = st_depth[sp];
    bool heap_sorted = false;
    while (last - first > kThreshold) {
      if (depth == 0) {
        if (lane == 0) std_heap_sort(e, first, last);
        heap_sorted = true;
        break;
      }
      --depth;
      const int mid = first + (last - first) / 2;
      if (lane == 0) std_move_median_to_first(e, first, first + 1, mid, last - 1);
      __syncthreads();
      const int cut = wave_unguarded_partition(e, first + 1, last, first, lp, rp, lane);
      const bool left = first < p1 && cut > p0;
      const bool right = cut < p1 && last > p0;
      if (left && right) {
        st_first[sp] = cut; st_last[sp] = last; st_depth[sp] = depth; ++sp;
        last = cut;
      } else if (right) {
        first = cut;
      } else {
        last = cut;
      }
    }
    if (!heap_sorted && lane == 0) std_insertion_sort(e, first, last);
    __syncthreads();
  }
}

// --- wave-parallel ATen row sum ------------------------------------------------------
// The vectorised inner sum above keeps 32 independent fp32 chains, accumulator k of lane
// e for k < 4, e < 8; each chain's adds (and the cascade that folds its levels) depend
// only on the unit counter.  Here each chain runs in its own wave lane (lane bits 3-4 = k,
// bits 0-2 = e) and the folds across chains happen in ATen's order through cross-lane
// reads, so every rounding is the one of the serial form.  The two half-waves sum with
// different RowViews (plain and required-masked).  Needs n >= 8; the result is returned
// in every lane of the half-wave.
__device__ __forceinline__ float aten_row_sum_wave(const RowView& r, int lane) {
  const int n = r.n;
  const int nunits = n / 8;
  const int half = lane >> 5, kq = (lane >> 3) & 3, e = lane & 7;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  const int size_ilp = nunits / 4;
  const int level_power = max(4, ceil_log2(size_ilp) / 4);
  const int level_step = 1 << level_power;
  const int level_mask = level_step - 1;
  int i = 0;
  while (i + level_step <= size_ilp) {
    for (int j = 0; j < level_step; ++j, ++i) a0 += r.at((i * 4 + kq) * 8 + e);
    a1 += a0;
    a0 = 0.f;
    if ((i & (level_mask << level_power)) == 0) {
      a2 += a1;
      a1 = 0.f;
      if ((i & (level_mask << (2 * level_power))) == 0) {
        a3 += a2;
        a2 = 0.f;
      }
    }
  }
  for (; i < size_ilp; ++i) a0 += r.at((i * 4 + kq) * 8 + e);
  a0 += a1;
  a0 += a2;
  a0 += a3;
  if (kq == 0)
    for (int v = size_ilp * 4; v < nunits; ++v) a0 += r.at(v * 8 + e);
  // Accumulators 1..3 into 0, in order (meaningful in the kq == 0 lanes).
  const float b1 = __shfl(a0, lane + 8), b2 = __shfl(a0, lane + 16), b3 = __shfl(a0, lane + 24);
  const float lane_sum = ((a0 + b1) + b2) + b3;
  float fin = 0.f;
  for (int t = nunits * 8; t < n; ++t) fin += r.at(t);
#pragma unroll
  for (int ee = 0; ee < 8; ++ee) fin += __shfl(lane_sum, (half << 5) + ee);
  return fin;
}

// --- cross-lane moves -------------------------------------------------------------------
// DPP controls (gfx9 encoding): quad_perm 0x00-0xff, row_shr:n 0x110+n, row_ror:n 0x120+n,
// row_bcast:15 0x142, row_bcast:31 0x143.  Lanes without a source (or outside ROW_MASK)
// keep `old`.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, 0xf, false);
}

// Inclusive scans over the 64 lanes: row_shr 1, 2, 4, 8 inside each 16-lane row, then the
// row totals carried by row_bcast:15 (into rows 1 and 3) and row_bcast:31 (rows 2 and 3).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ double dpp_f64_or_zero(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = dpp_u32<CTRL, ROW_MASK>(0u, (uint32_t)b);
  const uint32_t hi = dpp_u32<CTRL, ROW_MASK>(0u, (uint32_t)(b >> 32));
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double wave_scan_add_f64(double v) {
  v += dpp_f64_or_zero<0x111, 0xf>(v);
  v += dpp_f64_or_zero<0x112, 0xf>(v);
  v += dpp_f64_or_zero<0x114, 0xf>(v);
  v += dpp_f64_or_zero<0x118, 0xf>(v);
  v += dpp_f64_or_zero<0x142, 0xa>(v);
  v += dpp_f64_or_zero<0x143, 0xc>(v);
  return v;
}
__device__ __forceinline__ uint32_t wave_scan_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0x111, 0xf>(0u, v));
  v = max(v, dpp_u32<0x112, 0xf>(0u, v));
  v = max(v, dpp_u32<0x114, 0xf>(0u, v));
  v = max(v, dpp_u32<0x118, 0xf>(0u, v));
  v = max(v, dpp_u32<0x142, 0xa>(0u, v));
  v = max(v, dpp_u32<0x143, 0xc>(0u, v));
  return v;
}
__device__ __forceinline__ int wave_scan_min_i32(int v) {
  constexpr uint32_t kId = 0x7fffffffu;
  v = min(v, (int)dpp_u32<0x111, 0xf>(kId, (uint32_t)v));
  v = min(v, (int)dpp_u32<0x112, 0xf>(kId, (uint32_t)v));
  v = min(v, (int)dpp_u32<0x114, 0xf>(kId, (uint32_t)v));
  v = min(v, (int)dpp_u32<0x118, 0xf>(kId, (uint32_t)v));
  v = min(v, (int)dpp_u32<0x142, 0xa>(kId, (uint32_t)v));
  v = min(v, (int)dpp_u32<0x143, 0xc>(kId, (uint32_t)v));
  return v;
}

__device__ __forceinline__ double readlane_f64(double v, int l) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Value of lane `lane ^ M` (M = 1, 2, 4, 8: DPP; 16: ds_bpermute; 32: v_permlane32_swap).
// Every lane has a source under these controls, so plain DPP moves suffice.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xf, 0xf, false);
}

template <int M>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v, int lane) {
  if constexpr (M == 1) {
    return dpp_mov<0xb1>(v);  // quad_perm [1,0,3,2]
  } else if constexpr (M == 2) {
    return dpp_mov<0x4e>(v);  // quad_perm [2,3,0,1]
  } else if constexpr (M == 4) {
    const uint32_t up = dpp_mov<0x12c>(v);    // row_ror:12 -> lane + 4 (mod 16)
    const uint32_t down = dpp_mov<0x124>(v);  // row_ror:4  -> lane - 4 (mod 16)
    return (lane & 4) ? down : up;
  } else if constexpr (M == 8) {
    return dpp_mov<0x128>(v);  // row_ror:8 -> lane ^ 8
  } else if constexpr (M == 16) {
    return (uint32_t)__builtin_amdgcn_ds_bpermute((lane ^ 16) << 2, (int)v);
  } else {
    static_assert(M == 32, "lane distance");
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane & 32) ? r[0] : r[1];
  }
}

// --- bitonic sort keys ------------------------------------------------------------------
__device__ __forceinline__ uint32_t order_key(float x) {
  if (__builtin_isnan(x)) return 0xffffffffu;
  if (x == 0.f) x = 0.f;  // -0 and +0 compare equal
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ uint32_t order_key_inverse(uint32_t k) {
  if (k == 0xffffffffu) return 0x7fc00000u;  // NaN
  return (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
}

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src_lane_x4) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(src_lane_x4, (int)(uint32_t)v);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(src_lane_x4, (int)(uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}

// Descending bitonic sort of 256*C 32-bit order keys held in registers: key (c, r) of
// lane l is element j = c*256 + l*4 + r.  Distances 1 and 2 stay inside a lane, 4..128
// cross lanes, 256 and up cross a lane's own chunks.  A compare-exchange leaves the larger
// key at the lower index inside blocks whose `size` bit of j is clear and the smaller one
// where it is set, so the full network ends in descending order.  Only values are sorted:
// which of several equal keys lands where is never read (rows whose selection depends on
// the order of ties take the exact std::sort path).
template <int C, int D>
__device__ __forceinline__ void chunk_stage(uint32_t (&kk)[C][4], int size) {
#pragma unroll
  for (int c = 0; c < C; ++c) {
    if ((c & D) == 0) {
      const bool desc = ((c << 8) & size) == 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t x = kk[c][r], y = kk[c | D][r];
        const uint32_t hi = max(x, y), lo = min(x, y);
        kk[c][r] = desc ? hi : lo;
        kk[c | D][r] = desc ? lo : hi;
      }
    }
  }
}

// Distances 4..128: lane l pairs with lane l ^ M (M = distance / 4).
template <int C, int M>
__device__ __forceinline__ void xlane_stage(uint32_t (&kk)[C][4], int size, int lane) {
  const bool lo = (lane & M) == 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const bool desc = ((((c << 8) | (lane << 2))) & size) == 0;
    const bool want_max = lo == desc;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t x = kk[c][r];
      const uint32_t y = xor_lane<M>(x, lane);
      kk[c][r] = want_max ? max(x, y) : min(x, y);
    }
  }
}

// Distances 1 and 2: pairs inside a lane.
template <int C, int S>
__device__ __forceinline__ void lane_stage(uint32_t (&kk)[C][4], int size, int lane) {
#pragma unroll
  for (int c = 0; c < C; ++c) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if ((r & S) == 0) {
        const bool desc = ((((c << 8) | (lane << 2) | r)) & size) == 0;
        const uint32_t x = kk[c][r], y = kk[c][r | S];
        const uint32_t hi = max(x, y), lo = min(x, y);
        kk[c][r] = desc ? hi : lo;
        kk[c][r | S] = desc ? lo : hi;
      }
    }
  }
}

template <int C>
__device__ __forceinline__ void bitonic_sort_regs(uint32_t (&kk)[C][4], int lane) {
  constexpr int P = 256 * C;
  // Short networks are unrolled whole (every distance and direction a constant, no loop
  // or switch control on the scalar unit); long ones keep the loops to bound code size.
  constexpr int kUnrollSizes = C <= 2 ? 16 : 1;
  constexpr int kUnrollStrides = C <= 2 ? 8 : 1;
#pragma unroll kUnrollSizes
  for (int size = 2; size <= P; size <<= 1) {
    // Distances of 256 and up, longest first, each chunk distance a compile-time constant
    // (as separate steps rather than one indexed step, so every key stays in a register).
    if constexpr (C >= 16) {
      if (size >= 4096) chunk_stage<C, 8>(kk, size);
    }
    if constexpr (C >= 8) {
      if (size >= 2048) chunk_stage<C, 4>(kk, size);
    }
    if constexpr (C >= 4) {
      if (size >= 1024) chunk_stage<C, 2>(kk, size);
    }
    if constexpr (C >= 2) {
      if (size >= 512) chunk_stage<C, 1>(kk, size);
    }
#pragma unroll kUnrollStrides
    for (int stride = min(size >> 1, 128); stride >= 4; stride >>= 1) {
      switch (stride) {
        case 128: xlane_stage<C, 32>(kk, size, lane); break;
        case 64: xlane_stage<C, 16>(kk, size, lane); break;
        case 32: xlane_stage<C, 8>(kk, size, lane); break;
        case 16: xlane_stage<C, 4>(kk, size, lane); break;
        case 8: xlane_stage<C, 2>(kk, size, lane); break;
        default: xlane_stage<C, 1>(kk, size, lane); break;
      }
    }
    if (size >= 4) lane_stage<C, 2>(kk, size, lane);
    lane_stage<C, 1>(kk, size, lane);
  }
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const uint64_t o = shfl_u64(v, ((int)(threadIdx.x & 63) ^ m) << 2);
    v = o > v ? o : v;
  }
  return v;
}

// One 64-thread work-group per (head, query-block) row; rows of up to 256*C key blocks.
template <int C>
__global__ __launch_bounds__(64) void coverage_mask_kernel(MaskArgs a) {
  constexpr int NMAX = 256 * C;
  __shared__ float row[NMAX];
  __shared__ uint32_t keys[NMAX];                          // sorted order keys
  __shared__ __attribute__((aligned(16))) float sv[NMAX];  // sorted values
  __shared__ uint64_t pe[NMAX + 2];  // (value, index) entries in std::sort order, tie-exact rows
  __shared__ int stk[3 * 64];
  __shared__ int lrp[2 * NMAX];  // partition stop positions, tie-exact rows
  __shared__ uint8_t m[NMAX];
  __shared__ int k_sh, exact_sh, p0_sh, p1_sh;

  const int lane = threadIdx.x;
  const int rid = blockIdx.x;  // h * nq + qb
  const int qb = rid % a.nq;
  const int nk = a.nk;
  const float* src = a.scores + (int64_t)rid * nk;

  const bool video = a.mode == 1;
  const int tb = a.text_blocks;
  // Row segment that is sorted: joint -> whole row; video -> columns [tb, nk).
  const int off = video ? tb : 0;
  const int n = video ? max(nk - tb, 0) : nk;
  const bool video_row = video && qb >= tb && n > 0 && (a.nq - tb) > 0;

  // Row into LDS, all loads of a lane issued before the first store.
  {
    constexpr int NL = 4 * C;
    constexpr int NB = NL < 8 ? NL : 8;
#pragma unroll
    for (int i0 = 0; i0 < NL; i0 += NB) {
      float v[NB];
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int j = (i0 + u) * 64 + lane;
        v[u] = j < nk ? src[j] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int j = (i0 + u) * 64 + lane;
        if (j < nk) {
          row[j] = v[u];
          m[j] = ((qb < a.req_q) || (j < a.req_k)) ? 1 : 0;
        }
      }
    }
  }
  __syncthreads();

  // Sums: half-wave 0 the plain total, half-wave 1 the required-masked total (joint).
  float sum_plain = 0.f, sum_req = 0.f;
  if (!video || video_row) {
    RowView rv;
    rv.x = row + off;
    rv.n = n;
    rv.qb = qb;
    rv.req_q = a.req_q;
    rv.req_k = video ? 0 : a.req_k;
    rv.masked = (lane >= 32) && !video;
    float s;
    if (n >= 8) {
      s = aten_row_sum_wave(rv, lane);
    } else {
      float one[1];
      aten_units_sum<1>(rv, n, one);
      s = one[0];
    }
    sum_plain = __shfl(s, 0);
    sum_req = __shfl(s, 32);
  }

  const bool do_select = video ? video_row : true;
  float target = 0.f;
  int exact = 0;
  if (do_select) {
    float total = sum_plain;
    total = (total < 1e-6f) ? 1e-6f : total;  // clamp_min_ (NaN propagates)
    const float tgt = a.coverage * total;
    if (video) {
      target = tgt;
    } else {
      float res = tgt - sum_req;
      target = (res < 0.f) ? 0.f : res;
    }
    // Candidate order keys; positions past n hold 0, below every value's key.
    uint32_t kk[C][4];
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = c * 256 + lane * 4 + r;
        uint32_t key = 0u;
        if (j < n) {
          const bool req = !video && ((qb < a.req_q) || (j < a.req_k));
          key = order_key(req ? neg_inf() : row[off + j]);
        }
        kk[c][r] = key;
      }
    bitonic_sort_regs<C>(kk, lane);
#pragma unroll
    for (int c = 0; c < C; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = c * 256 + lane * 4 + r;
        keys[j] = kk[c][r];
        // The sorted value: -0 comes back as +0 and NaN as one NaN, neither of which
        // changes a prefix sum or its comparison with the target.
        if (j < n) sv[j] = __uint_as_float(order_key_inverse(kk[c][r]));
      }
    __syncthreads();

    // Prefix sums in fp64, each rounded to fp32: the first index reaching the target.
    // A prefix x[0..j] whose partial sums are all exact in fp64 gives the same sums in any
    // order: every partial sum is a multiple of 2^lsb_min (the lowest set bit over the
    // prefix) no larger than (j+1) * max|x| < 2^(ceil(log2(j+1)) + e(max|x|) + 1), exact
    // while that is at most 2^(lsb_min + 52).  Such prefixes are scanned 64 at a time
    // across the wave; from the first index past that bound (or a non-finite value) lane 0
    // continues the serial walk from the exact sum before it.
    int first = -1;
    {
      double base = 0.0;
      uint32_t run_max = 0u;    // max |x| (bits) so far
      int run_lsb = 0x7fffffff;  // lowest set-bit exponent so far
      int serial_from = -1;
      double serial_cum = 0.0;
      for (int c0 = 0; c0 < n; c0 += 64) {
        const int j = c0 + lane;
        float x = j < n ? sv[j] : 0.f;
        if (!video && !__builtin_isfinite(x)) x = 0.f;
        const uint32_t ab = __float_as_uint(x) & 0x7fffffffu;
        int lsb = 0x7fffffff;
        if (ab != 0u && ab < 0x7f800000u) {
          const uint32_t E = ab >> 23, mant = ab & 0x7fffffu;
          const uint32_t sig = E ? (mant | 0x800000u) : mant;
          lsb = (int)(E ? E : 1u) - 150 + __builtin_ctz(sig);
        }
        const uint32_t mx = max(run_max, wave_scan_max_u32(ab));
        const int mn = min(run_lsb, wave_scan_min_i32(lsb));
        bool ok;
        if (mx >= 0x7f800000u) {
          ok = false;  // inf or NaN in the prefix
        } else if (mx == 0u) {
          ok = true;
        } else {
          const int eM = (mx >> 23) ? (int)(mx >> 23) - 127 : -149 + (31 - __builtin_clz(mx));
          const int cl = j == 0 ? 0 : 32 - __builtin_clz((uint32_t)j);  // ceil(log2(j + 1))
          ok = cl + eM + 1 <= mn + 52;
        }
        const double S = base + wave_scan_add_f64((double)x);
        const bool valid = j < n;
        const uint64_t hits = __ballot(valid && ok && (float)S >= target);
        if (hits) {
          first = c0 + __builtin_ctzll(hits);
          break;
        }
        const uint64_t bad = __ballot(valid && !ok);
        if (bad) {
          const int f = __builtin_ctzll(bad);
          serial_from = c0 + f;
          serial_cum = f == 0 ? base : readlane_f64(S, f - 1);
          break;
        }
        base = readlane_f64(S, 63);
        run_max = (uint32_t)__builtin_amdgcn_readlane((int)mx, 63);
        run_lsb = __builtin_amdgcn_readlane(mn, 63);
      }
      if (serial_from >= 0 && lane == 0) {
        double cum = serial_cum;
        for (int i = serial_from; i < n; ++i) {
          float x = sv[i];
          if (!video && !__builtin_isfinite(x)) x = 0.f;
          cum += (double)x;
          if ((float)cum >= target) {
            first = i;
            break;
          }
        }
      }
    }
    if (lane == 0) {
      const int ncand = video ? n : ((qb < a.req_q) ? 0 : n - min(a.req_k, n));
      int k = target > 1e-6f ? (first >= 0 ? first + 1 : ncand) : 0;
      k = min(max(k, 0), n);
      int ex = 0;
      if (k > 0 && k < n && keys[k - 1] == keys[k]) ex = 1;
      k_sh = k;
      exact_sh = ex;
    }
    __syncthreads();
    exact = exact_sh;
  }

  const int k = do_select ? k_sh : 0;
  // Rows whose selection depends on the order of tied values: the tie group at the cut
  // occupies sorted positions [p0, p1) (keys equal to the k-th key), and std::sort's
  // order of exactly those positions decides which of its members are among the first k.
  if (do_select && exact) {
    if (lane == 0) {
      const uint32_t t = keys[k - 1];
      int lo = 0, hi = k - 1;  // first index whose key is not above t
      while (lo < hi) {
        const int md = (lo + hi) >> 1;
        if (keys[md] > t) lo = md + 1; else hi = md;
      }
      p0_sh = lo;
      lo = k + 1; hi = n;  // first index whose key is below t (keys[k] == t)
      while (lo < hi) {
        const int md = (lo + hi) >> 1;
        if (keys[md] >= t) lo = md + 1; else hi = md;
      }
      p1_sh = lo;
    }
    uint64_t* e = pe + 1;
    for (int j = lane; j < n; j += 64) {
      const bool req = !video && ((qb < a.req_q) || (j < a.req_k));
      e[j] = pmake(req ? neg_inf() : row[off + j], j);
    }
    __syncthreads();
    wave_sort_positions(e, n, p0_sh, p1_sh, stk, lrp, lrp + NMAX, lane);
  }

  if (exact) {
    // keys above the tie, then the tie group's members in std::sort order up to the cut
    const uint32_t t = keys[k - 1];
    for (int j = lane; j < n; j += 64) {
      const bool req = !video && ((qb < a.req_q) || (j < a.req_k));
      if (order_key(req ? neg_inf() : row[off + j]) > t) m[off + j] = 1;
    }
    for (int i = p0_sh + lane; i < k; i += 64) m[off + pidx(pe[1 + i])] = 1;
  } else if (k > 0) {
    // No tie straddles the cut: the first k of the sorted order are exactly the
    // candidates whose key is at least the k-th largest key.
    const uint32_t cut = keys[k - 1];
    for (int j = lane; j < n; j += 64) {
      const bool req = !video && ((qb < a.req_q) || (j < a.req_k));
      if (order_key(req ? neg_inf() : row[off + j]) >= cut) m[off + j] = 1;
    }
  }
  __syncthreads();
  if (!video && a.keep_diagonal && lane == 0 && qb < min(a.nq, nk)) m[qb] = 1;
  __syncthreads();

  // Row state for the empty-row fallback (applied by coverage_fixup_kernel once every
  // row is known): the empty flag, and whether the row's top-1 index depends on the order
  // of a tie at the top of the sort.
  int any = 0;
  for (int j = lane; j < nk; j += 64) any |= m[j];
  any = __any(any);
  uint8_t* mrow = a.mask + (int64_t)rid * nk;
  for (int j = lane; j < nk; j += 64) mrow[j] = m[j];
  // Joint rows whose top two keys are equal: their top-1 index depends on the order of
  // that tie, so the fallback takes it from the exact std::sort order.
  const int tie = (!video && n > 1 && keys[0] == keys[1]) ? 1 : 0;
  if (lane == 0) a.ws_flags[rid] = (uint8_t)((any ? 0 : 1) | (tie << 1));
}

// Phase 2, one 64-thread work-group per kFixupRows rows.  The reference's fallback
// `mask.scatter_(-1, top1, empty_rows.unsqueeze(-1))` (sparse_attention.py:327-330,
// 371-374) runs when ANY row of the tensor is empty and then sets mask[r, top1[r]] =
// empty[r] for EVERY row r -- it also clears the top-1 bit of non-empty rows.  Then the
// ascending index lists and counts of the final mask are written.
template <int C>
__global__ __launch_bounds__(64) void coverage_fixup_kernel(MaskArgs a) {
  constexpr int NMAX = 256 * C;
  __shared__ uint64_t pe[NMAX + 2];
  __shared__ int stk[3 * 64];
  __shared__ int lrp[2 * NMAX];
  __shared__ uint8_t m[NMAX];
  const int lane = threadIdx.x;
  const int rows = a.H * a.nq;
  const int nk = a.nk;
  // Empty flags (bit 0 of each byte), four rows per 32-bit word; the flag region is
  // padded to 256 bytes, and bytes past `rows` are masked off.
  uint32_t any_empty = 0;
  {
    const uint32_t* fw = reinterpret_cast<const uint32_t*>(a.ws_flags);
    const int words = (rows + 3) >> 2;
    for (int w0 = 0; w0 < words; w0 += 64 * 8) {
      uint32_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int w = w0 + u * 64 + lane;
        v[u] = w < words ? fw[w] : 0u;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int w = w0 + u * 64 + lane;
        const int left = rows - 4 * w;  // rows held by this word
        const uint32_t keep = left >= 4 ? 0x01010101u : (left == 3 ? 0x010101u : (left == 2 ? 0x0101u : 0x01u));
        any_empty |= v[u] & keep;
      }
    }
  }
  const bool fallback = __any(any_empty != 0);
  if (!fallback && a.idx == nullptr && a.counts == nullptr) return;  // the mask is final
  // kFixupRows rows per work-group share the one scan of the flags above.
  const int rid_end = (int)min((int64_t)rows, ((int64_t)blockIdx.x + 1) * kFixupRows);
  for (int rid = (int)blockIdx.x * kFixupRows; rid < rid_end; ++rid) {
    const int qb = rid % a.nq;
    uint8_t* mrow = a.mask + (int64_t)rid * nk;
    for (int j = lane; j < nk; j += 64) m[j] = mrow[j];
    __syncthreads();
    if (fallback) {
      // Top-1: video -> scores.argmax(dim=-1) over the full row, the first NaN if there is
      // one, else the first maximum (-0 == +0); joint -> sorted_indices[..., 0], the
      // candidate of the largest key, from the exact std::sort order when the top two keys
      // tie.  Without such a tie both are the largest (order_key, ~index) pair of the row.
      const uint8_t flags = a.ws_flags[rid];
      const float* src = a.scores + (int64_t)rid * nk;
      const bool video = a.mode == 1;
      int t;
      if (flags & 2) {
        uint64_t* e = pe + 1;
        for (int j = lane; j < nk; j += 64) {
          const bool req = (qb < a.req_q) || (j < a.req_k);
          e[j] = pmake(req ? neg_inf() : src[j], j);
        }
        __syncthreads();
        wave_sort_positions(e, nk, 0, 1, stk, lrp, lrp + NMAX, lane);
        t = pidx(pe[1]);
      } else {
        uint64_t best = 0ull;
        for (int j = lane; j < nk; j += 64) {
          const bool req = !video && ((qb < a.req_q) || (j < a.req_k));
          const uint64_t key = ((uint64_t)order_key(req ? neg_inf() : src[j]) << 32) | (uint64_t)(~(uint32_t)j);
          best = key > best ? key : best;
        }
        best = wave_max_u64(best);
        t = (int)(~(uint32_t)(best & 0xffffffffull));
      }
      if (lane == 0) {
        m[t] = flags & 1;
        mrow[t] = flags & 1;
      }
      __syncthreads();
    }
    if (a.idx != nullptr || a.counts != nullptr) {
      int base = 0;
      for (int c0 = 0; c0 < nk; c0 += 64) {
        const int j = c0 + lane;
        const bool on = j < nk && m[j];
        const uint64_t bal = __ballot(on);
        if (on && a.idx != nullptr)
          a.idx[(int64_t)rid * nk + base + __popcll(bal & ((1ull << lane) - 1ull))] = j;
        base += __popcll(bal);
      }
      if (lane == 0 && a.counts != nullptr) a.counts[rid] = base;
    }
    __syncthreads();  // m is refilled for the next row
  }
}

template <int C>
static hipError_t launch_mask_c(const MaskArgs& a, int rows, hipStream_t stream) {
  coverage_mask_kernel<C><<<rows, 64, 0, stream>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  coverage_fixup_kernel<C><<<(int)(((int64_t)rows + kFixupRows - 1) / kFixupRows), 64, 0, stream>>>(a);
  return hipGetLastError();
}

hipError_t launch_coverage_mask(const MaskArgs& a, hipStream_t stream) {
  const int rows = a.H * a.nq;
  if (rows == 0 || a.nk == 0) return hipSuccess;
  if (a.nk > kMaskMaxN) return hipErrorInvalidValue;
  if (a.nk <= 256) return launch_mask_c<1>(a, rows, stream);
  if (a.nk <= 512) return launch_mask_c<2>(a, rows, stream);
  if (a.nk <= 1024) return launch_mask_c<4>(a, rows, stream);
  if (a.nk <= 2048) return launch_mask_c<8>(a, rows, stream);
  return launch_mask_c<16>(a, rows, stream);
}

}  // namespace sa
