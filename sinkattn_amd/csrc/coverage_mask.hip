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
// One 64-thread work-group handles one (head, query-block) row.  The row is sorted with
// a bitonic network keyed (value desc, index asc).  Values, prefix sums and the cut k
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

// Row capacities: rows of up to 1024 key blocks use the small instance (21 KB of LDS),
// longer rows (up to 4096) the large one (84 KB, one work-group per CU).
constexpr int kMaskSmallN = 1024;
constexpr int kMaskMaxN = 4096;

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
struct PairArr {
  float* v;
  int* id;
  __device__ __forceinline__ bool comp(int a, int b) const {  // element a before b
    const float x = v[a], y = v[b];
    return (__builtin_isnan(x) && !__builtin_isnan(y)) || (x > y);
  }
  __device__ __forceinline__ bool comp_val(float x, int b) const {
    const float y = v[b];
    return (__builtin_isnan(x) && !__builtin_isnan(y)) || (x > y);
  }
  __device__ __forceinline__ bool comp_val2(int a, float y) const {
    const float x = v[a];
    return (__builtin_isnan(x) && !__builtin_isnan(y)) || (x > y);
  }
  __device__ __forceinline__ void swap(int a, int b) const {
    const float tv = v[a]; v[a] = v[b]; v[b] = tv;
    const int ti = id[a]; id[a] = id[b]; id[b] = ti;
  }
};

__device__ void std_move_median_to_first(const PairArr& p, int result, int a, int b, int c) {
  if (p.comp(a, b)) {
    if (p.comp(b, c)) p.swap(result, b);
    else if (p.comp(a, c)) p.swap(result, c);
    else p.swap(result, a);
  } else if (p.comp(a, c)) {
    p.swap(result, a);
  } else if (p.comp(b, c)) {
    p.swap(result, c);
  } else {
    p.swap(result, b);
  }
}

__device__ int std_unguarded_partition(const PairArr& p, int first, int last, int pivot) {
  while (true) {
    while (p.comp(first, pivot)) ++first;
    --last;
    while (p.comp(pivot, last)) --last;
    if (!(first < last)) return first;
    p.swap(first, last);
    ++first;
  }
}

// __adjust_heap(first, hole, len, value) on [base, base+len)
__device__ void std_adjust_heap(const PairArr& p, int base, int hole, int len, float val, int vid) {
  const int top = hole;
  int second = hole;
  while (second < (len - 1) / 2) {
    second = 2 * (second + 1);
    if (p.comp(base + second, base + second - 1)) second--;
    p.v[base + hole] = p.v[base + second];
    p.id[base + hole] = p.id[base + second];
    hole = second;
  }
  if ((len & 1) == 0 && second == (len - 2) / 2) {
    second = 2 * (second + 1);
    p.v[base + hole] = p.v[base + second - 1];
    p.id[base + hole] = p.id[base + second - 1];
    hole = second - 1;
  }
  // __push_heap
  int parent = (hole - 1) / 2;
  while (hole > top && p.comp_val2(base + parent, val)) {
    p.v[base + hole] = p.v[base + parent];
    p.id[base + hole] = p.id[base + parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  p.v[base + hole] = val;
  p.id[base + hole] = vid;
}

__device__ void std_heap_sort(const PairArr& p, int first, int last) {
  const int len = last - first;
  if (len >= 2) {  // __make_heap
    int parent = (len - 2) / 2;
    while (true) {
      const float val = p.v[first + parent];
      const int vid = p.id[first + parent];
      std_adjust_heap(p, first, parent, len, val, vid);
      if (parent == 0) break;
      parent--;
    }
  }
  // __sort_heap
  while (last - first > 1) {
    --last;
    const float val = p.v[last];
    const int vid = p.id[last];
    p.v[last] = p.v[first];
    p.id[last] = p.id[first];
    std_adjust_heap(p, first, 0, last - first, val, vid);
  }
}

__device__ void std_unguarded_linear_insert(const PairArr& p, int last) {
  const float val = p.v[last];
  const int vid = p.id[last];
  int next = last - 1;
  while (p.comp_val(val, next)) {
    p.v[last] = p.v[next];
    p.id[last] = p.id[next];
    last = next;
    --next;
  }
  p.v[last] = val;
  p.id[last] = vid;
}

__device__ void std_insertion_sort(const PairArr& p, int first, int last) {
  if (first == last) return;
  for (int i = first + 1; i != last; ++i) {
    if (p.comp(i, first)) {
      const float val = p.v[i];
      const int vid = p.id[i];
      for (int j = i; j > first; --j) {
        p.v[j] = p.v[j - 1];
        p.id[j] = p.id[j - 1];
      }
      p.v[first] = val;
      p.id[first] = vid;
    } else {
      std_unguarded_linear_insert(p, i);
    }
  }
}

__device__ void std_sort(const PairArr& p, int n) {
  if (n <= 1) return;
  constexpr int kThreshold = 16;
  // __introsort_loop with an explicit stack: [first, last, depth]
  int st_first[64], st_last[64], st_depth[64];
  int sp = 0;
  st_first[sp] = 0; st_last[sp] = n; st_depth[sp] = 2 * (31 - __clz(n)); ++sp;
  while (sp > 0) {
    --sp;
    int first = st_first[sp], last = st_last[sp], depth = st_depth[sp];
    while (last - first > kThreshold) {
      if (depth == 0) {
        std_heap_sort(p, first, last);
        break;
      }
      --depth;
      const int mid = first + (last - first) / 2;
      std_move_median_to_first(p, first, first + 1, mid, last - 1);
      const int cut = std_unguarded_partition(p, first + 1, last, first);
      st_first[sp] = cut; st_last[sp] = last; st_depth[sp] = depth; ++sp;
      last = cut;
    }
  }
  // __final_insertion_sort
  if (n > kThreshold) {
    std_insertion_sort(p, 0, kThreshold);
    for (int i = kThreshold; i < n; ++i) std_unguarded_linear_insert(p, i);
  } else {
    std_insertion_sort(p, 0, n);
  }
}

// --- bitonic sort keys ------------------------------------------------------------------
__device__ __forceinline__ uint32_t order_key(float x) {
  if (__builtin_isnan(x)) return 0xffffffffu;
  if (x == 0.f) x = 0.f;  // -0 and +0 compare equal
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

template <int NMAX>
__global__ __launch_bounds__(64) void coverage_mask_kernel(MaskArgs a) {
  __shared__ float row[NMAX];
  __shared__ unsigned long long keys[NMAX];
  __shared__ float sv[NMAX];    // sorted values (tie-exact order when needed)
  __shared__ int si[NMAX];      // sorted indices
  __shared__ uint8_t m[NMAX];
  __shared__ float sums_sh[2];
  __shared__ int k_sh, exact_sh;

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

  for (int j = lane; j < nk; j += 64) {
    row[j] = src[j];
    const bool req = (qb < a.req_q) || (j < a.req_k);
    m[j] = req ? 1 : 0;
  }
  __syncthreads();

  // Sums: lane 0 plain total, lane 1 required-masked total (joint) -- same code path.
  if (lane < 2) {
    RowView rv;
    rv.x = row + off;
    rv.n = n;
    rv.qb = qb;
    rv.req_q = a.req_q;
    rv.req_k = video ? 0 : a.req_k;
    rv.masked = (lane == 1) && !video;
    const float s = (!video || video_row) ? aten_row_sum(rv) : 0.f;
    sums_sh[lane] = s;
  }
  __syncthreads();

  const bool do_select = video ? video_row : true;
  float target = 0.f;
  if (do_select) {
    float total = sums_sh[0];
    total = (total < 1e-6f) ? 1e-6f : total;  // clamp_min_ (NaN propagates)
    const float tgt = a.coverage * total;
    if (video) {
      target = tgt;
    } else {
      float res = tgt - sums_sh[1];
      target = (res < 0.f) ? 0.f : res;
    }
    // Candidate keys.
    int P = 1;
    while (P < n) P <<= 1;
    for (int j = lane; j < P; j += 64) {
      unsigned long long key = 0ull;
      if (j < n) {
        const float x = row[off + j];
        const bool req = !video && ((qb < a.req_q) || (j < a.req_k));
        const float cv = req ? neg_inf() : x;
        key = ((unsigned long long)order_key(cv) << 32) | (unsigned long long)(~(uint32_t)j);
      }
      keys[j] = key;
    }
    __syncthreads();
    // Bitonic sort, descending.
    for (int size = 2; size <= P; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int t = lane; t < P / 2; t += 64) {
          const int lo = 2 * t - (t & (stride - 1));
          const int hi = lo + stride;
          const bool desc = ((lo & size) == 0);
          const unsigned long long x = keys[lo], y = keys[hi];
          if ((x < y) == desc) {
            keys[lo] = y;
            keys[hi] = x;
          }
        }
        __syncthreads();
      }
    }
    for (int j = lane; j < n; j += 64) {
      const int id = (int)(~(uint32_t)(keys[j] & 0xffffffffull));
      si[j] = id;
      const bool req = !video && ((qb < a.req_q) || (id < a.req_k));
      sv[j] = req ? neg_inf() : row[off + id];
    }
    __syncthreads();

    if (lane == 0) {
      // Prefix sums in fp64, each rounded to fp32, first index reaching the target.
      double cum = 0.0;
      int first = -1;
      for (int i = 0; i < n; ++i) {
        float x = sv[i];
        if (!video && !__builtin_isfinite(x)) x = 0.f;
        cum += (double)x;
        if (first < 0 && (float)cum >= target) first = i;
      }
      int ncand = 0;
      if (video) {
        ncand = n;
      } else {
        for (int j = 0; j < n; ++j) ncand += ((qb < a.req_q) || (j < a.req_k)) ? 0 : 1;
      }
      int k = target > 1e-6f ? (first >= 0 ? first + 1 : ncand) : 0;
      k = min(max(k, 0), n);
      int exact = 0;
      if (k > 0 && k < n && (keys[k - 1] >> 32) == (keys[k] >> 32)) exact = 1;
      k_sh = k;
      exact_sh = exact;
    }
    __syncthreads();
  }

  const int k = do_select ? k_sh : 0;
  // Exact permutation for rows whose selection depends on the order of tied values.
  auto run_exact = [&]() {
    if (lane == 0) {
      for (int j = 0; j < n; ++j) {
        const bool req = !video && ((qb < a.req_q) || (j < a.req_k));
        sv[j] = req ? neg_inf() : row[off + j];
        si[j] = j;
      }
      PairArr p{sv, si};
      std_sort(p, n);
    }
    __syncthreads();
  };
  if (do_select && exact_sh) run_exact();

  for (int i = lane; i < k; i += 64) m[off + si[i]] = 1;
  __syncthreads();
  if (!video && a.keep_diagonal && lane == 0 && qb < min(a.nq, nk)) m[qb] = 1;
  __syncthreads();

  // Row state for the empty-row fallback (applied by coverage_fixup_kernel once every
  // row is known): empty flag, top-1 index, and whether that index still depends on the
  // order of a tie at the top of the sort.
  int any = 0;
  for (int j = lane; j < nk; j += 64) any |= m[j];
  any = __any(any);
  uint8_t* mrow = a.mask + (int64_t)rid * nk;
  for (int j = lane; j < nk; j += 64) mrow[j] = m[j];
  if (lane == 0) {
    int top1 = 0, tie = 0;
    if (video) {  // scores.argmax(dim=-1): first maximum of the full row, NaN maximal
      float bv = row[0];
      for (int j = 1; j < nk; ++j) {
        const float x = row[j];
        if (__builtin_isnan(bv)) break;
        if (__builtin_isnan(x) || x > bv) { bv = x; top1 = j; }
      }
    } else {  // sorted_indices[..., 0]
      top1 = si[0];
      tie = (!exact_sh && n > 1 && (keys[0] >> 32) == (keys[1] >> 32)) ? 1 : 0;
    }
    a.ws_top1[rid] = top1;
    a.ws_flags[rid] = (uint8_t)((any ? 0 : 1) | (tie << 1));
  }
}

// Phase 2, one 64-thread work-group per row.  The reference's fallback
// `mask.scatter_(-1, top1, empty_rows.unsqueeze(-1))` (sparse_attention.py:327-330,
// 371-374) runs when ANY row of the tensor is empty and then sets mask[r, top1[r]] =
// empty[r] for EVERY row r -- it also clears the top-1 bit of non-empty rows.  Then the
// ascending index lists and counts of the final mask are written.
template <int NMAX>
__global__ __launch_bounds__(64) void coverage_fixup_kernel(MaskArgs a) {
  __shared__ float sv[NMAX];
  __shared__ int si[NMAX];
  __shared__ uint8_t m[NMAX];
  const int lane = threadIdx.x;
  const int rid = blockIdx.x;
  const int rows = a.H * a.nq;
  const int qb = rid % a.nq;
  const int nk = a.nk;
  int any_empty = 0;
  for (int i = lane; i < rows; i += 64) any_empty |= a.ws_flags[i] & 1;
  any_empty = __any(any_empty);
  uint8_t* mrow = a.mask + (int64_t)rid * nk;
  for (int j = lane; j < nk; j += 64) m[j] = mrow[j];
  __syncthreads();
  if (any_empty) {
    const uint8_t flags = a.ws_flags[rid];
    if (lane == 0) {
      int t = a.ws_top1[rid];
      if (flags & 2) {  // joint branch, tie at the top: exact std::sort order
        const float* src = a.scores + (int64_t)rid * nk;
        for (int j = 0; j < nk; ++j) {
          const bool req = (qb < a.req_q) || (j < a.req_k);
          sv[j] = req ? neg_inf() : src[j];
          si[j] = j;
        }
        PairArr p{sv, si};
        std_sort(p, nk);
        t = si[0];
      }
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
}

hipError_t launch_coverage_mask(const MaskArgs& a, hipStream_t stream) {
  const int rows = a.H * a.nq;
  if (rows == 0 || a.nk == 0) return hipSuccess;
  if (a.nk <= kMaskSmallN) {
    coverage_mask_kernel<kMaskSmallN><<<rows, 64, 0, stream>>>(a);
  } else {
    coverage_mask_kernel<kMaskMaxN><<<rows, 64, 0, stream>>>(a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.nk <= kMaskSmallN) {
    coverage_fixup_kernel<kMaskSmallN><<<rows, 64, 0, stream>>>(a);
  } else {
    coverage_fixup_kernel<kMaskMaxN><<<rows, 64, 0, stream>>>(a);
  }
  return hipGetLastError();
}

}  // namespace sa
