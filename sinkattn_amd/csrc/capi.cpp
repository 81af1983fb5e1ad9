// extern "C" entry points of libsinkattn (declared in include/sinkattn.h): argument
// validation, then a stream-ordered launch.  Nothing here allocates device memory.

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/sinkattn.h"
#include "kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return -1;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return 0;
  g_last_error = std::string(what) + ": " + hipGetErrorString(e);
  return (int)e;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool valid_dtype(int dt) { return dt == SINKATTN_BF16 || dt == SINKATTN_F16 || dt == SINKATTN_F32; }

// BHSD operand: innermost stride 1, 16-byte aligned base, outer strides multiples of 8.
int check_operand(const char* name, const void* p, const int64_t* s) {
  if (p == nullptr) return fail("%s: null pointer", name);
  if (s == nullptr) return fail("%s: null strides", name);
  if (s[3] != 1) return fail("%s: innermost stride must be 1 (got %lld)", name, (long long)s[3]);
  if (reinterpret_cast<uintptr_t>(p) % 16 != 0) return fail("%s: base must be 16-byte aligned", name);
  for (int i = 0; i < 3; ++i)
    if (s[i] % 8 != 0 || s[i] < 0)
      return fail("%s: stride[%d]=%lld must be a non-negative multiple of 8 elements", name, i,
                  (long long)s[i]);
  return 0;
}

const int64_t kMaxInt = 0x7fffffffLL;

}  // namespace

namespace sa {

int api_fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return -1;
}

int api_hip_status(hipError_t e, const char* what) { return hip_status(e, what); }

}  // namespace sa

extern "C" {

const char* sinkattn_last_error(void) { return g_last_error.c_str(); }

int sinkattn_abi_version(void) { return 4; }

int64_t sinkattn_block_sparse_order_slots(int64_t B, int64_t H, int64_t nqb) {
  if (B <= 0 || H <= 0 || nqb <= 0 || B * H * nqb > kMaxInt) return 0;
  return sa::plan_order_slots((int)(B * H * nqb), (int)nqb);
}

int64_t sinkattn_block_sparse_order_cache_ints(int64_t B, int64_t H, int64_t nqb, int64_t entries) {
  if (B <= 0 || H <= 0 || nqb <= 0 || B * H * nqb > kMaxInt || entries < 1 || entries > 4096) return 0;
  return sa::plan_order_cache_ints((int)(B * H * nqb), (int)nqb, (int)entries);
}

static int plan_impl(const uint8_t* mask, const int64_t mask_strides[4], int64_t B, int64_t H,
                     int64_t nqb, int64_t nkb, int32_t* counts, int32_t* idx, int32_t* order,
                     int32_t* cache, int64_t entries, void* stream) {
  if (B < 0 || H < 0 || nqb < 0 || nkb < 0) return fail("plan: negative size");
  const int64_t rows = B * H * nqb;
  if (rows > kMaxInt || nkb > 8192) return fail("plan: too many rows or key blocks (nkb <= 8192)");
  if (rows == 0) return 0;
  if (mask == nullptr || mask_strides == nullptr || counts == nullptr || idx == nullptr)
    return fail("plan: null pointer");
  if (cache != nullptr && (order == nullptr || entries < 1 || entries > 4096))
    return fail("plan: a launch-order cache needs an order buffer and 1..4096 entries");
  sa::PlanArgs a{};
  a.mask = mask;
  for (int i = 0; i < 4; ++i) a.ms[i] = mask_strides[i];
  a.H = (int)H;
  a.nqb = (int)nqb;
  a.nkb = (int)nkb;
  a.rows = (int)rows;
  a.counts = counts;
  a.idx = idx;
  a.order = order;
  a.cache = cache;
  a.cache_entries = cache != nullptr ? (int)entries : 0;
  return hip_status(sa::launch_block_sparse_plan(a, (hipStream_t)stream), "plan launch");
}

int sinkattn_block_sparse_plan(const uint8_t* mask, const int64_t mask_strides[4], int64_t B,
                               int64_t H, int64_t nqb, int64_t nkb, int32_t* counts,
                               int32_t* idx, int32_t* order, void* stream) {
  return plan_impl(mask, mask_strides, B, H, nqb, nkb, counts, idx, order, nullptr, 0, stream);
}

int sinkattn_block_sparse_plan_cached(const uint8_t* mask, const int64_t mask_strides[4], int64_t B,
                                      int64_t H, int64_t nqb, int64_t nkb, int32_t* counts,
                                      int32_t* idx, int32_t* order, int32_t* order_cache,
                                      int64_t cache_entries, void* stream) {
  if (order_cache == nullptr) return fail("plan_cached: null launch-order cache");
  return plan_impl(mask, mask_strides, B, H, nqb, nkb, counts, idx, order, order_cache, cache_entries,
                   stream);
}

}  // extern "C"

namespace {

struct CompTiles {
  const void* kd = nullptr;
  const void* vd = nullptr;
  const int64_t* kds = nullptr;
  const int64_t* vds = nullptr;
  int64_t Nd = 0, qblocks = 0;
  float log_gap = 0.f;
};

int block_sparse_fwd_impl(const void* q, const void* k, const void* v, int dtype, int64_t B,
                          int64_t H, int64_t Nq, int64_t Nk, int64_t D, const int64_t q_strides[4],
                          const int64_t k_strides[4], const int64_t v_strides[4], void* out,
                          const int64_t out_strides[4], float* lse, const int32_t* counts,
                          const int32_t* idx, const int32_t* order, int64_t nqb, int64_t nkb,
                          float softmax_scale, const CompTiles& comp, void* stream) {
  if (!valid_dtype(dtype)) return fail("fwd: unsupported dtype %d", dtype);
  if (D != 32 && D != 64 && D != 128) return fail("fwd: head dim %lld not supported (32, 64 or 128)", (long long)D);
  if (B < 0 || H < 0 || Nq < 0 || Nk < 0) return fail("fwd: negative size");
  if (nqb != cdiv(Nq, 128) || nkb != cdiv(Nk, 128))
    return fail("fwd: plan is [%lld,%lld] blocks, expected [%lld,%lld]", (long long)nqb,
                (long long)nkb, (long long)cdiv(Nq, 128), (long long)cdiv(Nk, 128));
  if (B * H * nqb > kMaxInt || Nq > kMaxInt || Nk > kMaxInt) return fail("fwd: sizes exceed int32");
  if (B * H * nqb == 0) return 0;
  int rc;
  if ((rc = check_operand("q", q, q_strides)) != 0) return rc;
  if ((rc = check_operand("k", k, k_strides)) != 0) return rc;
  if ((rc = check_operand("v", v, v_strides)) != 0) return rc;
  if ((rc = check_operand("out", out, out_strides)) != 0) return rc;
  if (counts == nullptr || idx == nullptr) return fail("fwd: null plan");
  if (dtype != SINKATTN_F32 && D == 128) {
    if (k_strides[2] < D || v_strides[2] < D) return fail("fwd: k/v row stride below the head dim");
    if (Nk * k_strides[2] * 2 >= (int64_t)1 << 31 || Nk * v_strides[2] * 2 >= (int64_t)1 << 31)
      return fail("fwd: one head of k or v spans more than 2 GiB");
  }
  sa::FwdArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.lse = lse;
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q_strides[i];
    a.ks[i] = k_strides[i];
    a.vs[i] = v_strides[i];
    a.os[i] = out_strides[i];
  }
  a.counts = counts;
  a.idx = idx;
  a.order = order;
  a.B = (int)B;
  a.H = (int)H;
  a.Nq = (int)Nq;
  a.Nk = (int)Nk;
  a.nqb = (int)nqb;
  a.nkb = (int)nkb;
  a.scale = softmax_scale;
  if (comp.qblocks > 0 && comp.Nd > 0) {
    if (dtype == SINKATTN_F32 || D != 128) return fail("fwd_comp: compensation tiles need bf16/f16 and D=128");
    if (comp.qblocks > nqb) return fail("fwd_comp: comp_qblocks %lld exceeds %lld q-blocks", (long long)comp.qblocks, (long long)nqb);
    if (comp.Nd > kMaxInt) return fail("fwd_comp: Nd exceeds int32");
    if ((rc = check_operand("kd", comp.kd, comp.kds)) != 0) return rc;
    if ((rc = check_operand("vd", comp.vd, comp.vds)) != 0) return rc;
    if (comp.kds[2] != k_strides[2] || comp.vds[2] != v_strides[2])
      return fail("fwd_comp: kd/vd row strides must equal k/v row strides");
    if (comp.Nd * k_strides[2] * 2 >= (int64_t)1 << 31 || comp.Nd * v_strides[2] * 2 >= (int64_t)1 << 31)
      return fail("fwd_comp: one head of kd or vd spans more than 2 GiB");
    if (!(comp.log_gap >= 0.f) || comp.log_gap > 64.f) return fail("fwd_comp: log_gap %g out of range", comp.log_gap);
    a.kd = comp.kd;
    a.vd = comp.vd;
    a.kds[0] = comp.kds[0];
    a.kds[1] = comp.kds[1];
    a.vds[0] = comp.vds[0];
    a.vds[1] = comp.vds[1];
    a.Nd = (int)comp.Nd;
    a.comp_qblocks = (int)comp.qblocks;
    a.comp_bias = comp.log_gap * 1.4426950408889634f;
  }
  return hip_status(sa::launch_block_sparse_fwd(a, dtype, (int)D, (hipStream_t)stream), "fwd launch");
}

}  // namespace

extern "C" {

int sinkattn_block_sparse_fwd(const void* q, const void* k, const void* v, int dtype, int64_t B,
                              int64_t H, int64_t Nq, int64_t Nk, int64_t D,
                              const int64_t q_strides[4], const int64_t k_strides[4],
                              const int64_t v_strides[4], void* out,
                              const int64_t out_strides[4], float* lse, const int32_t* counts,
                              const int32_t* idx, const int32_t* order, int64_t nqb, int64_t nkb,
                              float softmax_scale, void* stream) {
  return block_sparse_fwd_impl(q, k, v, dtype, B, H, Nq, Nk, D, q_strides, k_strides, v_strides, out,
                               out_strides, lse, counts, idx, order, nqb, nkb, softmax_scale, CompTiles{},
                               stream);
}

int sinkattn_block_sparse_fwd_comp(const void* q, const void* k, const void* v, int dtype, int64_t B,
                                   int64_t H, int64_t Nq, int64_t Nk, int64_t D,
                                   const int64_t q_strides[4], const int64_t k_strides[4],
                                   const int64_t v_strides[4], const void* kd, const void* vd,
                                   const int64_t kd_strides[4], const int64_t vd_strides[4], int64_t Nd,
                                   int64_t comp_qblocks, float log_gap, void* out,
                                   const int64_t out_strides[4], float* lse, const int32_t* counts,
                                   const int32_t* idx, const int32_t* order, int64_t nqb, int64_t nkb,
                                   float softmax_scale, void* stream) {
  if (comp_qblocks < 0 || Nd < 0) return fail("fwd_comp: negative size");
  CompTiles comp;
  comp.kd = kd;
  comp.vd = vd;
  comp.kds = kd_strides;
  comp.vds = vd_strides;
  comp.Nd = Nd;
  comp.qblocks = comp_qblocks;
  comp.log_gap = log_gap;
  return block_sparse_fwd_impl(q, k, v, dtype, B, H, Nq, Nk, D, q_strides, k_strides, v_strides, out,
                               out_strides, lse, counts, idx, order, nqb, nkb, softmax_scale, comp, stream);
}

int64_t sinkattn_mean_pool_tokens_rows(int64_t N, int64_t prefix, int64_t gap) {
  if (N < 0 || gap < 1) return -1;
  if (gap == 1) return N;
  const int64_t p = prefix < 0 ? 0 : (prefix > N ? N : prefix);
  if (p >= N) return N;
  return p + cdiv(N - p, gap);
}

int sinkattn_mean_pool_tokens(const void* x, int dtype, int64_t B, int64_t H, int64_t N, int64_t D,
                              const int64_t x_strides[4], int64_t prefix, int64_t gap, void* out,
                              const int64_t out_strides[4], void* stream) {
  if (!valid_dtype(dtype)) return fail("mean_pool_tokens: unsupported dtype %d", dtype);
  if (B < 0 || H < 0 || N < 0 || gap < 1) return fail("mean_pool_tokens: bad size or gap");
  const int64_t es = dtype == SINKATTN_F32 ? 4 : 2;
  const int64_t chunks = D * es / 16;
  if (D <= 0 || (D * es) % 16 != 0 || chunks > 256 || (chunks & (chunks - 1)) != 0)
    return fail("mean_pool_tokens: head dim %lld unsupported (row of 16..4096 bytes, power of two)", (long long)D);
  const int64_t nout = sinkattn_mean_pool_tokens_rows(N, prefix, gap);
  if (B * H > 65535 || N > kMaxInt) return fail("mean_pool_tokens: sizes exceed the launch limits");
  if (B * H * nout == 0) return 0;
  int rc;
  if ((rc = check_operand("x", x, x_strides)) != 0) return rc;
  if ((rc = check_operand("out", out, out_strides)) != 0) return rc;
  sa::TokenPoolArgs a{};
  a.x = x;
  a.out = out;
  for (int i = 0; i < 4; ++i) {
    a.xs[i] = x_strides[i];
    a.os[i] = out_strides[i];
  }
  a.B = (int)B;
  a.H = (int)H;
  a.N = (int)N;
  a.D = (int)D;
  a.Nout = (int)nout;
  a.gap = gap == 1 ? 1 : (int)gap;
  const int64_t p = prefix < 0 ? 0 : (prefix > N ? N : prefix);
  a.prefix = (gap == 1 || p >= N) ? (int)N : (int)p;  // identity cases copy every row
  return hip_status(sa::launch_mean_pool_tokens(a, dtype, (hipStream_t)stream), "mean_pool_tokens launch");
}

int sinkattn_qk_norm_rotary(const void* q_in, const void* k_in, int dtype, int64_t rows, int64_t C,
                            int64_t D, int64_t in_row_stride, const float* wq, const float* wk, float eps_q,
                            float eps_k, const float* freq_real, const float* freq_imag, int64_t rows_per_pos,
                            int64_t freq_rows, void* q_out, void* k_out, int64_t out_row_stride, void* stream) {
  if (!valid_dtype(dtype)) return fail("qk_norm_rotary: unsupported dtype %d", dtype);
  const int64_t epc = dtype == SINKATTN_F32 ? 4 : 8;
  if (rows < 0 || C <= 0 || D <= 0 || C % D != 0 || D % epc != 0 || C / epc > 1024)
    return fail("qk_norm_rotary: C=%lld, D=%lld unsupported (D | C, D a multiple of %lld, C <= %lld)",
                (long long)C, (long long)D, (long long)epc, (long long)(1024 * epc));
  if (rows == 0) return 0;
  if (rows_per_pos < 1 || freq_rows < 1) return fail("qk_norm_rotary: bad rotation table indexing");
  if (in_row_stride < C || out_row_stride < C || in_row_stride % epc || out_row_stride % epc)
    return fail("qk_norm_rotary: row strides must be >= C and multiples of 16 bytes");
  if ((rows + 3) / 4 > kMaxInt) return fail("qk_norm_rotary: too many rows");
  const void* ptrs[6] = {q_in, k_in, q_out, k_out, wq, wk};
  for (const void* p : ptrs)
    if (p == nullptr || reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return fail("qk_norm_rotary: tensors and weights must be non-null and 16-byte aligned");
  if ((freq_real == nullptr) != (freq_imag == nullptr)) return fail("qk_norm_rotary: give both or neither table");
  if (freq_real != nullptr && (reinterpret_cast<uintptr_t>(freq_real) % 16 != 0 ||
                               reinterpret_cast<uintptr_t>(freq_imag) % 16 != 0))
    return fail("qk_norm_rotary: rotation tables must be 16-byte aligned");
  sa::QkPrepArgs a{};
  a.q_in = q_in;
  a.k_in = k_in;
  a.q_out = q_out;
  a.k_out = k_out;
  a.in_stride = in_row_stride;
  a.out_stride = out_row_stride;
  a.wq = wq;
  a.wk = wk;
  a.eps_q = eps_q;
  a.eps_k = eps_k;
  a.freq_real = freq_real;
  a.freq_imag = freq_imag;
  a.rows = rows;
  a.rows_per_pos = rows_per_pos;
  a.freq_rows = freq_rows;
  a.C = (int)C;
  a.D = (int)D;
  return hip_status(sa::launch_qk_prep(a, dtype, (hipStream_t)stream), "qk_norm_rotary launch");
}

int sinkattn_lse_mix(const void* sink_out, const int64_t sink_strides[4], const void* sink_lse,
                     const int64_t sink_lse_strides[3], const void* dyn_out, const int64_t dyn_strides[4],
                     const void* dyn_lse, const int64_t dyn_lse_strides[3], int dtype, int64_t B, int64_t H,
                     int64_t N, int64_t D, float log_gap, void* out, const int64_t out_strides[4],
                     void* stream) {
  if (!valid_dtype(dtype)) return fail("lse_mix: unsupported dtype %d", dtype);
  if (B < 0 || H < 0 || N < 0) return fail("lse_mix: negative size");
  const int64_t es = dtype == SINKATTN_F32 ? 4 : 2;
  if (D <= 0 || (D * es) % 16 != 0) return fail("lse_mix: head dim %lld unsupported (multiple of 16 bytes)", (long long)D);
  if (B * H * N * (D * es / 16) > ((int64_t)1 << 40)) return fail("lse_mix: too large");
  if (B * H * N == 0) return 0;
  int rc;
  if ((rc = check_operand("sink_out", sink_out, sink_strides)) != 0) return rc;
  if ((rc = check_operand("dyn_out", dyn_out, dyn_strides)) != 0) return rc;
  if ((rc = check_operand("out", out, out_strides)) != 0) return rc;
  if (sink_lse == nullptr || dyn_lse == nullptr || sink_lse_strides == nullptr || dyn_lse_strides == nullptr)
    return fail("lse_mix: null lse");
  sa::MixArgs a{};
  a.sink = sink_out;
  a.dyn = dyn_out;
  a.lse_s = sink_lse;
  a.lse_d = dyn_lse;
  a.out = out;
  for (int i = 0; i < 4; ++i) {
    a.ss[i] = sink_strides[i];
    a.ds[i] = dyn_strides[i];
    a.os[i] = out_strides[i];
  }
  for (int i = 0; i < 3; ++i) {
    a.lss[i] = sink_lse_strides[i];
    a.lds[i] = dyn_lse_strides[i];
  }
  a.B = (int)B;
  a.H = (int)H;
  a.N = (int)N;
  a.D = (int)D;
  a.log_gap = log_gap;
  return hip_status(sa::launch_lse_mix(a, dtype, (hipStream_t)stream), "lse_mix launch");
}

static int fill_pool_args(sa::PoolArgs& a, const char* who, const void* q, const void* k, int dtype,
                          int64_t B, int64_t H, int64_t Hk, int64_t Nq, int64_t Nk, int64_t D,
                          const int64_t* qs, const int64_t* ks, int64_t block_size) {
  if (!valid_dtype(dtype)) return fail("%s: unsupported dtype %d", who, dtype);
  if (block_size < 1 || block_size > 1024)
    return fail("%s: block_size %lld not supported (1..1024)", who, (long long)block_size);
  if (D < 1 || D > 1024) return fail("%s: head dim %lld not supported", who, (long long)D);
  if (B < 0 || H < 0 || Hk <= 0 || Nq < 0 || Nk < 0) return fail("%s: bad size", who);
  if (H % Hk != 0) return fail("%s: query heads %lld not a multiple of kv heads %lld", who, (long long)H, (long long)Hk);
  if (Nq > kMaxInt || Nk > kMaxInt || B * H * cdiv(Nq, 128) > kMaxInt) return fail("%s: sizes exceed int32", who);
  int rc;
  if (B * H * Nq > 0) {
    if ((rc = check_operand("q", q, qs)) != 0) return rc;
    if ((rc = check_operand("k", k, ks)) != 0) return rc;
  }
  a.q = q;
  a.k = k;
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = qs[i];
    a.ks[i] = ks[i];
  }
  a.B = (int)B;
  a.H = (int)H;
  a.Hk = (int)Hk;
  a.Nq = (int)Nq;
  a.Nk = (int)Nk;
  a.nqb = (int)cdiv(Nq, block_size);
  a.nkb = (int)cdiv(Nk, block_size);
  a.bs = (int)block_size;
  a.D = (int)D;
  return 0;
}

// The generic pooling kernels (any block size and head dim) hold a query-row group, a key
// tile, a score tile and one map row in LDS.
static int check_generic_pool(const char* who, const sa::PoolArgs& a, int dtype) {
  if (a.D > 256) return fail("%s: head dim %d above 256 needs block_size 128 and head dim 128", who, a.D);
  if (sa::generic_pool_lds_need(a.D, a.nkb, dtype) > sa::kGenericPoolMaxLds)
    return fail("%s: %d key blocks of head dim %d exceed the generic kernel's LDS", who, a.nkb, a.D);
  return 0;
}

// Block sizes the persistent matrix-core block-mass kernel takes (head dim 128, 16-bit).
static bool mass_mfma_block(int64_t block_size) {
  return block_size == 16 || block_size == 32 || block_size == 64 || block_size == 128;
}

size_t sinkattn_block_mass_pool_workspace_bytes(int64_t B, int64_t H, int64_t Nq, int64_t Nk,
                                                int64_t block_size, int dtype) {
  if (dtype == SINKATTN_F32 || !mass_mfma_block(block_size)) return 0;
  const int64_t items = B * H * cdiv(Nq, 128);  // items of 128 query rows
  const int64_t groups = items < sa::block_mass_groups() ? items : sa::block_mass_groups();
  return (size_t)(groups * cdiv(Nk, block_size) * 128 * (int64_t)sizeof(float));
}

int sinkattn_block_mass_pool(const void* q, const void* k, int dtype, int64_t B, int64_t H,
                             int64_t Nq, int64_t Nk, int64_t D, const int64_t q_strides[4],
                             const int64_t k_strides[4], int64_t block_size, float scale,
                             float* out, void* workspace, void* stream) {
  sa::PoolArgs a{};
  int rc = fill_pool_args(a, "block_mass_pool", q, k, dtype, B, H, H, Nq, Nk, D, q_strides,
                          k_strides, block_size);
  if (rc != 0) return rc;
  if (Nk == 0) return fail("block_mass_pool: no keys");
  if (out == nullptr) return fail("block_mass_pool: null output");
  a.scale = scale;
  a.out = out;
  a.ws = reinterpret_cast<float*>(workspace);
  const bool at128 = block_size == 128 && D == 128;
  if (mass_mfma_block(block_size) && D == 128 && dtype != SINKATTN_F32) {  // persistent MFMA kernel, workspace slots
    if (workspace == nullptr) return fail("block_mass_pool: null workspace");
    if (k_strides[2] < D) return fail("block_mass_pool: k row stride below the head dim");
    if (Nk * k_strides[2] * 2 >= (int64_t)1 << 31)
      return fail("block_mass_pool: one head of k spans more than 2 GiB");
    return hip_status(sa::launch_block_mass_pool(a, dtype, (int)D, (hipStream_t)stream), "pool launch");
  }
  if (at128 && a.nkb <= 256)  // fp32 MFMA kernel
    return hip_status(sa::launch_block_mass_pool(a, dtype, (int)D, (hipStream_t)stream), "pool launch");
  if ((rc = check_generic_pool("block_mass_pool", a, dtype)) != 0) return rc;
  return hip_status(sa::launch_block_mass_generic(a, dtype, (hipStream_t)stream), "pool launch");
}

size_t sinkattn_max_pool_workspace_bytes(int64_t B, int64_t H, int64_t N, int64_t block_size, int dtype) {
  if (dtype == SINKATTN_F32 || !mass_mfma_block(block_size)) return 0;
  const int64_t items = B * H * cdiv(N, 128);  // items of 128 query rows
  const int64_t groups = items < sa::max_pool_groups() ? items : sa::max_pool_groups();
  // per group: the rows' block maxima, and below block 128 the item's column maxima
  const int64_t per_kb = 128 + (block_size == 128 ? 0 : 128 / block_size);
  return (size_t)(groups * cdiv(N, block_size) * per_kb * (int64_t)sizeof(float));
}

int sinkattn_max_pool(const void* q, const void* k, int dtype, int64_t B, int64_t H, int64_t Hk,
                      int64_t N, int64_t D, const int64_t q_strides[4], const int64_t k_strides[4],
                      int64_t block_size, float sm_scale, int causal, void* po, void* workspace,
                      void* stream) {
  sa::PoolArgs a{};
  int rc = fill_pool_args(a, "max_pool", q, k, dtype, B, H, Hk, N, N, D, q_strides, k_strides,
                          block_size);
  if (rc != 0) return rc;
  // the reference's asserts (pooling_kernel.py:198-207)
  if (block_size != 16 && block_size != 32 && block_size != 64 && block_size != 128)
    return fail("max_pool: block_size %lld not in {16, 32, 64, 128}", (long long)block_size);
  if (D != 16 && D != 32 && D != 64 && D != 128 && D != 256)
    return fail("max_pool: head dim %lld not in {16, 32, 64, 128, 256}", (long long)D);
  if (B * H * N == 0) return 0;
  if (po == nullptr) return fail("max_pool: null output");
  a.scale = sm_scale;
  a.causal = causal ? 1 : 0;
  a.out = po;
  a.ws = static_cast<float*>(workspace);
  if (dtype != SINKATTN_F32 && D == 128 && (block_size != 128 || a.nkb <= 1024)) {
    // persistent MFMA kernel, workspace slots
    if (workspace == nullptr) return fail("max_pool: null workspace (see sinkattn_max_pool_workspace_bytes)");
    if (k_strides[2] < D || N * k_strides[2] * 2 >= (int64_t)1 << 31)
      return fail("max_pool: k row stride below the head dim or one head of k over 2 GiB");
    return hip_status(sa::launch_max_pool(a, dtype, (int)D, (hipStream_t)stream), "max_pool launch");
  }
  if ((rc = check_generic_pool("max_pool", a, dtype)) != 0) return rc;
  return hip_status(sa::launch_max_pool_generic(a, dtype, (hipStream_t)stream), "max_pool launch");
}

size_t sinkattn_mean_pool_workspace_bytes(int64_t B, int64_t H, int64_t Nq, int64_t Nk, int64_t D,
                                          int64_t block_size) {
  if (block_size <= 0) return 0;
  return (size_t)(B * H * (cdiv(Nq, block_size) + cdiv(Nk, block_size)) * D) * sizeof(float);
}

int sinkattn_mean_pool_scores(const void* q, const void* k, int dtype, int64_t B, int64_t H,
                              int64_t Nq, int64_t Nk, int64_t D, const int64_t q_strides[4],
                              const int64_t k_strides[4], int64_t block_size, float scale,
                              void* workspace, float* out, void* stream) {
  sa::PoolArgs a{};
  int rc = fill_pool_args(a, "mean_pool", q, k, dtype, B, H, H, Nq, Nk, D, q_strides, k_strides,
                          block_size);
  if (rc != 0) return rc;
  if (Nq == 0 || Nk == 0) return fail("mean_pool: empty sequence");
  if (workspace == nullptr || out == nullptr) return fail("mean_pool: null workspace or output");
  a.scale = scale;
  a.out = out;
  a.ws = reinterpret_cast<float*>(workspace);
  return hip_status(sa::launch_mean_pool(a, dtype, (int)D, (hipStream_t)stream), "mean_pool launch");
}

size_t sinkattn_coverage_mask_workspace_bytes(int64_t H, int64_t nq) {
  const int64_t rows = H * nq > 0 ? H * nq : 0;
  return (size_t)(((rows + 255) / 256) * 256);
}

int sinkattn_coverage_mask(const float* scores, int64_t H, int64_t nq, int64_t nk, float coverage,
                           int keep_diagonal, int64_t req_q, int64_t req_k, int mode,
                           int64_t text_blocks, uint8_t* mask, int32_t* counts, int32_t* idx,
                           void* workspace, void* stream) {
  if (H < 0 || nq < 0 || nk < 0) return fail("coverage_mask: negative size");
  if (nk > 4096) return fail("coverage_mask: %lld key blocks exceed the supported 4096", (long long)nk);
  if (H * nq > kMaxInt) return fail("coverage_mask: too many rows");
  if (mode != 0 && mode != 1) return fail("coverage_mask: mode must be 0 (joint) or 1 (video_residual)");
  if (req_q < 0 || req_k < 0 || text_blocks < 0) return fail("coverage_mask: negative block count");
  if (H * nq * nk == 0) return 0;
  if (scores == nullptr || mask == nullptr || workspace == nullptr)
    return fail("coverage_mask: null pointer");
  sa::MaskArgs a{};
  a.scores = scores;
  a.H = (int)H;
  a.nq = (int)nq;
  a.nk = (int)nk;
  a.coverage = coverage;
  a.keep_diagonal = keep_diagonal ? 1 : 0;
  a.req_q = (int)(req_q < nq ? req_q : nq);
  a.req_k = (int)(req_k < nk ? req_k : nk);
  a.mode = mode;
  a.text_blocks = (int)text_blocks;
  a.mask = mask;
  a.counts = counts;
  a.idx = idx;
  a.ws_flags = reinterpret_cast<uint8_t*>(workspace);
  return hip_status(sa::launch_coverage_mask(a, (hipStream_t)stream), "coverage_mask launch");
}

}  // extern "C"
