/*
 * TEST INFRASTRUCTURE ONLY (parity oracle).  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this; the product never does.
 *
 * Plain-C restatement of the reference's coverage-mask builder
 * `_build_direct_mean_coverage_mask` (sinkattention/sparse_attention.py:268-376) together
 * with the CPU torch arithmetic it inherits:
 *   - oracle_aten_row_sum: fp32 row sum in ATen's order (vectorized_inner_sum ->
 *     row_sum -> multi_row_sum with 8-lane vectors, 4 accumulators, 4 cascade levels;
 *     rows shorter than 8 take scalar_inner_sum, the same scheme on scalars);
 *   - oracle_cumsum_f32: fp64-accumulated prefix sums rounded to fp32 (torch.cumsum);
 *   - oracle_std_sort_desc: libstdc++ std::sort (introsort, threshold 16, median of
 *     three, heap-sort fallback, final insertion sort) on (value, index) pairs with the
 *     comparator (isnan(a) && !isnan(b)) || a > b, i.e. torch.sort(descending=True);
 *   - oracle_coverage_mask: both branches (joint / video_residual) of the builder plus
 *     `_build_offline_required_mask` (:241-265).
 * Pinned in tests/test_oracle_coverage.py against torch on this machine and against a
 * real libstdc++ std::sort (oracle/stdsort_ref.cpp).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int ceil_log2_i64(int64_t v) {
  int r = 0;
  if (v <= 1) return 0;
  v -= 1;
  while (v > 0) {
    v >>= 1;
    r++;
  }
  return r;
}

/* ATen's row_sum over `nunits` units of L lanes (L = 8: fp32 vectors, L = 1: scalars):
 * multi_row_sum with 4 interleaved accumulators and 4 cascade levels, leftover units
 * added to accumulator 0, then accumulators folded 0+1+2+3.  Result per lane in out[]. */
static void aten_units_sum(const float* x, int64_t nunits, int L, float* out) {
  enum { ILP = 4, LEVELS = 4, LMAX = 8 };
  const int64_t size_ilp = nunits / ILP;
  float acc[LEVELS][ILP][LMAX];
  memset(acc, 0, sizeof(acc));
  int level_power = ceil_log2_i64(size_ilp) / LEVELS;
  if (level_power < 4) level_power = 4;
  const int64_t level_step = (int64_t)1 << level_power;
  const int64_t level_mask = level_step - 1;
  int64_t i = 0;
  while (i + level_step <= size_ilp) {
    for (int64_t j = 0; j < level_step; ++j, ++i)
      for (int k = 0; k < ILP; ++k)
        for (int e = 0; e < L; ++e) acc[0][k][e] += x[(i * ILP + k) * L + e];
    for (int j = 1; j < LEVELS; ++j) {
      for (int k = 0; k < ILP; ++k)
        for (int e = 0; e < L; ++e) {
          acc[j][k][e] += acc[j - 1][k][e];
          acc[j - 1][k][e] = 0.f;
        }
      if ((i & (level_mask << (j * level_power))) != 0) break;
    }
  }
  for (; i < size_ilp; ++i)
    for (int k = 0; k < ILP; ++k)
      for (int e = 0; e < L; ++e) acc[0][k][e] += x[(i * ILP + k) * L + e];
  for (int j = 1; j < LEVELS; ++j)
    for (int k = 0; k < ILP; ++k)
      for (int e = 0; e < L; ++e) acc[0][k][e] += acc[j][k][e];
  for (int64_t v = size_ilp * ILP; v < nunits; ++v)
    for (int e = 0; e < L; ++e) acc[0][0][e] += x[v * L + e];
  for (int k = 1; k < ILP; ++k)
    for (int e = 0; e < L; ++e) acc[0][0][e] += acc[0][k][e];
  for (int e = 0; e < L; ++e) out[e] = acc[0][0][e];
}

/* Contiguous fp32 row sum in ATen's order: rows of at least 8 elements take the
 * vectorised inner sum (8-lane units, then the scalar tail summed from 0 and the lanes
 * added in order); shorter rows take the scalar inner sum. */
float oracle_aten_row_sum(const float* x, int64_t n) {
  float lanes[8];
  if (n < 8) {
    aten_units_sum(x, n, 1, lanes);
    return lanes[0];
  }
  const int64_t vec_size = n / 8;
  aten_units_sum(x, vec_size, 8, lanes);
  float fin = 0.f;
  for (int64_t t = vec_size * 8; t < n; ++t) fin += x[t];
  for (int e = 0; e < 8; ++e) fin += lanes[e];
  return fin;
}

void oracle_cumsum_f32(const float* x, int64_t n, float* out) {
  double c = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    c += (double)x[i];
    out[i] = (float)c;
  }
}

/* ---- libstdc++ std::sort on (value, index) pairs ---------------------------------- */
typedef struct {
  float* v;
  int64_t* id;
} pairs_t;

static int cmp_vals(float x, float y) { return (isnan(x) && !isnan(y)) || (x > y); }
static int cmp(const pairs_t* p, int64_t a, int64_t b) { return cmp_vals(p->v[a], p->v[b]); }
static void swp(const pairs_t* p, int64_t a, int64_t b) {
  float tv = p->v[a];
  int64_t ti = p->id[a];
  p->v[a] = p->v[b];
  p->id[a] = p->id[b];
  p->v[b] = tv;
  p->id[b] = ti;
}
static void mov(const pairs_t* p, int64_t dst, int64_t src) {
  p->v[dst] = p->v[src];
  p->id[dst] = p->id[src];
}

static void move_median_to_first(const pairs_t* p, int64_t r, int64_t a, int64_t b, int64_t c) {
  if (cmp(p, a, b)) {
    if (cmp(p, b, c)) swp(p, r, b);
    else if (cmp(p, a, c)) swp(p, r, c);
    else swp(p, r, a);
  } else if (cmp(p, a, c)) {
    swp(p, r, a);
  } else if (cmp(p, b, c)) {
    swp(p, r, c);
  } else {
    swp(p, r, b);
  }
}

static int64_t unguarded_partition(const pairs_t* p, int64_t first, int64_t last, int64_t pivot) {
  for (;;) {
    while (cmp(p, first, pivot)) ++first;
    --last;
    while (cmp(p, pivot, last)) --last;
    if (!(first < last)) return first;
    swp(p, first, last);
    ++first;
  }
}

static void adjust_heap(const pairs_t* p, int64_t base, int64_t hole, int64_t len, float val,
                        int64_t vid) {
  const int64_t top = hole;
  int64_t child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (cmp(p, base + child, base + child - 1)) child--;
    mov(p, base + hole, base + child);
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    mov(p, base + hole, base + child - 1);
    hole = child - 1;
  }
  int64_t parent = (hole - 1) / 2;
  while (hole > top && cmp_vals(p->v[base + parent], val)) {
    mov(p, base + hole, base + parent);
    hole = parent;
    parent = (hole - 1) / 2;
  }
  p->v[base + hole] = val;
  p->id[base + hole] = vid;
}

static void heap_sort(const pairs_t* p, int64_t first, int64_t last) {
  const int64_t len = last - first;
  if (len >= 2) {
    int64_t parent = (len - 2) / 2;
    for (;;) {
      adjust_heap(p, first, parent, len, p->v[first + parent], p->id[first + parent]);
      if (parent == 0) break;
      parent--;
    }
  }
  while (last - first > 1) {
    --last;
    float val = p->v[last];
    int64_t vid = p->id[last];
    mov(p, last, first);
    adjust_heap(p, first, 0, last - first, val, vid);
  }
}

static void introsort_loop(const pairs_t* p, int64_t first, int64_t last, int64_t depth) {
  while (last - first > 16) {
    if (depth == 0) {
      heap_sort(p, first, last);
      return;
    }
    --depth;
    int64_t mid = first + (last - first) / 2;
    move_median_to_first(p, first, first + 1, mid, last - 1);
    int64_t cut = unguarded_partition(p, first + 1, last, first);
    introsort_loop(p, cut, last, depth);
    last = cut;
  }
}

static void unguarded_linear_insert(const pairs_t* p, int64_t last) {
  float val = p->v[last];
  int64_t vid = p->id[last];
  int64_t next = last - 1;
  while (cmp_vals(val, p->v[next])) {
    mov(p, last, next);
    last = next;
    --next;
  }
  p->v[last] = val;
  p->id[last] = vid;
}

static void insertion_sort(const pairs_t* p, int64_t first, int64_t last) {
  if (first == last) return;
  for (int64_t i = first + 1; i != last; ++i) {
    if (cmp(p, i, first)) {
      float val = p->v[i];
      int64_t vid = p->id[i];
      for (int64_t j = i; j > first; --j) mov(p, j, j - 1);
      p->v[first] = val;
      p->id[first] = vid;
    } else {
      unguarded_linear_insert(p, i);
    }
  }
}

static int64_t lg(int64_t n) {
  int64_t r = -1;
  while (n > 0) {
    n >>= 1;
    r++;
  }
  return r;
}

void oracle_std_sort_desc(float* v, int64_t* id, int64_t n) {
  pairs_t p = {v, id};
  if (n <= 1) return;
  introsort_loop(&p, 0, n, 2 * lg(n));
  if (n > 16) {
    insertion_sort(&p, 0, 16);
    for (int64_t i = 16; i < n; ++i) unguarded_linear_insert(&p, i);
  } else {
    insertion_sort(&p, 0, n);
  }
}

/* ---- the builder -------------------------------------------------------------------- */
/* Builds one row up to (not including) the empty-row fallback; returns the row's first
 * index in sort order (its "top1") and whether the row is empty. */
static void coverage_row_joint(const float* s, int64_t nk, int64_t qb, int64_t nq, float cov,
                               int keep_diag, int64_t req_q, int64_t req_k, uint8_t* m,
                               float* wv, int64_t* wi, float* wtmp, int64_t* top1, int* empty) {
  for (int64_t j = 0; j < nk; ++j) m[j] = (qb < req_q) || (j < req_k);
  float total = oracle_aten_row_sum(s, nk);
  if (total < 1e-6f) total = 1e-6f;
  for (int64_t j = 0; j < nk; ++j) wtmp[j] = s[j] * (m[j] ? 1.f : 0.f);
  const float selected = oracle_aten_row_sum(wtmp, nk);
  const float target = cov * total;
  float res = target - selected;
  if (res < 0.f) res = 0.f;
  int64_t ncand = 0;
  for (int64_t j = 0; j < nk; ++j) {
    wv[j] = m[j] ? -INFINITY : s[j];
    wi[j] = j;
    ncand += m[j] ? 0 : 1;
  }
  oracle_std_sort_desc(wv, wi, nk);
  for (int64_t j = 0; j < nk; ++j) wtmp[j] = isfinite(wv[j]) ? wv[j] : 0.f;
  double c = 0.0;
  int64_t first = -1;
  for (int64_t j = 0; j < nk; ++j) {
    c += (double)wtmp[j];
    if (first < 0 && (float)c >= res) first = j;
  }
  int64_t k = res > 1e-6f ? (first >= 0 ? first + 1 : ncand) : 0;
  if (k < 0) k = 0;
  if (k > nk) k = nk;
  for (int64_t i = 0; i < k; ++i) m[wi[i]] = 1;
  if (keep_diag && qb < (nq < nk ? nq : nk)) m[qb] = 1;
  int any = 0;
  for (int64_t j = 0; j < nk; ++j) any |= m[j];
  *empty = !any;
  *top1 = wi[0];
}

static void coverage_row_video(const float* s, int64_t nk, int64_t qb, int64_t nq, float cov,
                               int64_t req_q, int64_t req_k, int64_t tb, uint8_t* m, float* wv,
                               int64_t* wi, int64_t* top1, int* empty) {
  for (int64_t j = 0; j < nk; ++j) m[j] = (qb < req_q) || (j < req_k);
  const int64_t nvid = nk - tb;
  if (qb >= tb && nvid > 0 && nq - tb > 0) {
    const float* vs = s + tb;
    float total = oracle_aten_row_sum(vs, nvid);
    if (total < 1e-6f) total = 1e-6f;
    const float target = cov * total;
    for (int64_t j = 0; j < nvid; ++j) {
      wv[j] = vs[j];
      wi[j] = j;
    }
    oracle_std_sort_desc(wv, wi, nvid);
    double c = 0.0;
    int64_t first = -1;
    for (int64_t j = 0; j < nvid; ++j) {
      c += (double)wv[j];
      if (first < 0 && (float)c >= target) first = j;
    }
    int64_t k = target > 1e-6f ? (first >= 0 ? first + 1 : nvid) : 0;
    if (k < 0) k = 0;
    if (k > nvid) k = nvid;
    for (int64_t i = 0; i < k; ++i) m[tb + wi[i]] = 1;
  }
  int any = 0;
  for (int64_t j = 0; j < nk; ++j) any |= m[j];
  /* top1 = scores.argmax(dim=-1): first maximum of the full row, NaN maximal */
  int64_t best = 0;
  for (int64_t j = 1; j < nk; ++j) {
    if (isnan(s[best])) break;
    if (isnan(s[j]) || s[j] > s[best]) best = j;
  }
  *empty = !any;
  *top1 = best;
}

/* scores fp32 [H, nq, nk] contiguous -> mask uint8 [H, nq, nk].  mode 0 = joint,
 * 1 = video_residual with tb leading text blocks.
 * The empty-row fallback is the reference's `mask.scatter_(-1, top1, empty_rows)`
 * (sparse_attention.py:327-330, 371-374): when any row of the whole tensor is empty,
 * every row r gets mask[r, top1[r]] = empty[r] -- which also CLEARS the top1 bit of
 * the non-empty rows.  Reproduced as is. */
void oracle_coverage_mask(const float* scores, int64_t H, int64_t nq, int64_t nk, float cov,
                          int keep_diag, int64_t req_q, int64_t req_k, int mode, int64_t tb,
                          uint8_t* out) {
  float* wv = (float*)malloc(sizeof(float) * (size_t)(nk > 0 ? nk : 1));
  float* wtmp = (float*)malloc(sizeof(float) * (size_t)(nk > 0 ? nk : 1));
  int64_t* wi = (int64_t*)malloc(sizeof(int64_t) * (size_t)(nk > 0 ? nk : 1));
  const int64_t rows = H * nq;
  int64_t* top1 = (int64_t*)malloc(sizeof(int64_t) * (size_t)(rows > 0 ? rows : 1));
  int* empty = (int*)malloc(sizeof(int) * (size_t)(rows > 0 ? rows : 1));
  int any_empty = 0;
  for (int64_t h = 0; h < H; ++h)
    for (int64_t qb = 0; qb < nq; ++qb) {
      const int64_t r = h * nq + qb;
      const float* s = scores + r * nk;
      uint8_t* m = out + r * nk;
      if (mode == 0)
        coverage_row_joint(s, nk, qb, nq, cov, keep_diag, req_q, req_k, m, wv, wi, wtmp, &top1[r], &empty[r]);
      else
        coverage_row_video(s, nk, qb, nq, cov, req_q, req_k, tb, m, wv, wi, &top1[r], &empty[r]);
      any_empty |= empty[r];
    }
  if (any_empty && nk > 0)
    for (int64_t r = 0; r < rows; ++r) out[r * nk + top1[r]] = (uint8_t)empty[r];
  free(top1);
  free(empty);
  free(wv);
  free(wtmp);
  free(wi);
}
