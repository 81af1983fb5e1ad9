/*
 * libsinkattn — MI355X (gfx950) kernels for SinkAttention's sparse-attention hot path.
 *
 * C ABI: plain device pointers, int64 shapes, element strides, a hipStream_t passed as
 * void*.  Every entry point returns an int status:
 *     0            success (work is enqueued on `stream`, nothing is synchronised)
 *    <0            invalid argument (nothing was enqueued); see sinkattn_last_error()
 *    >0            a hipError_t from a launch
 * No C++ exception crosses this boundary and no entry point allocates device memory:
 * outputs and workspaces are supplied by the caller (sizes from the *_bytes queries).
 * All work is stream-ordered.  Every function is stateless and reentrant except
 * sinkattn_block_sparse_attn_noalloc (end of this file): it keeps its plan in one static
 * device array per GPU (SINKATTN_NOALLOC_SCRATCH_BYTES = 32 MiB, reserved on every GPU
 * that loads this library, whether or not that entry point is called), so calls of it that
 * overlap on one GPU race.  sinkattn_block_sparse_plan_cached keeps state only in the
 * launch-order cache buffer its caller passes (calls sharing one buffer must be ordered).
 *
 * Tensor conventions.  A "BHSD" operand is addressed as
 *     base[b*s[0] + h*s[1] + n*s[2] + d*s[3]]   with s[3] == 1,
 * so both contiguous [B,H,N,D] tensors and [B,N,H,D] memory viewed as [B,H,N,D]
 * (what the reference's varlen call produces) are accepted without copies.
 * Vector loads need the base 16-byte aligned and s[0..2] multiples of 8 elements.
 *
 * The reference (bb-2020-bb/sinkattn) is Python; the citations below name the Python
 * function each entry point replaces.
 */
#ifndef SINKATTN_H_
#define SINKATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of Q/K/V/O. */
enum sinkattn_dtype { SINKATTN_BF16 = 0, SINKATTN_F16 = 1, SINKATTN_F32 = 2 };

/* Message for the last non-zero status returned on the calling thread ("" if none). */
const char* sinkattn_last_error(void);

/* ABI version of this library (bumped on any change of a signature or of a buffer's
 * contract; 3: the order buffer of a plan also holds its chunk table; 4: plans with a
 * launch-order cache). */
int sinkattn_abi_version(void);

/* ------------------------------------------------------------------------------------
 * Block-sparse plan: bool block mask -> per-(b,h,q-block) ascending key-block lists.
 *
 * Replaces the mask hand-off of `_block_sparse_attn` -> `block_sparse_attn_func(...,
 * base_blockmask=block_mask.contiguous(), ...)` (sinkattention/sparse_attention.py:743,762):
 * the external kernel consumed the bool mask directly; here it is turned once into
 *   counts[B*H*nqb]          number of listed key blocks per row,
 *   idx[B*H*nqb*nkb]         the listed key blocks of row r in idx[r*nkb .. r*nkb+counts[r]),
 *   order[n]                 n = sinkattn_block_sparse_order_slots() int32 entries: the
 *                            launch slots (work-group i, on XCD i % 8, runs row order[i];
 *                            -1: none), then a chunk table the plan uses internally.
 *                            Each head's q-blocks go to the XCDs in chunks (longest-
 *                            processing-time first over the XCDs, long rows leading each
 *                            XCD's sequence), so an XCD's L2 holds few heads' K/V at once.
 * `mask` is uint8/bool [B,H,nqb,nkb] with element strides mask_strides[4].
 * ---------------------------------------------------------------------------------- */
int64_t sinkattn_block_sparse_order_slots(int64_t B, int64_t H, int64_t nqb);
int sinkattn_block_sparse_plan(const uint8_t* mask, const int64_t mask_strides[4],
                               int64_t B, int64_t H, int64_t nqb, int64_t nkb,
                               int32_t* counts, int32_t* idx, int32_t* order,
                               void* stream);

/* ------------------------------------------------------------------------------------
 * Block-sparse plan with a launch-order cache.
 *
 * Replaces the same hand-off as sinkattn_block_sparse_plan, for callers that hand the
 * forward a freshly built mask tensor on every call, as the reference's Z-Image processor
 * does (zimg/runtime/sink_sparse_zimage.py:513-538: `_slice_runtime_sink_mask` +
 * `_force_text_dense_runtime_mask` per sample per call).  The lists and counts are always
 * built from `mask`; the launch order, which depends only on the shape and the per-row
 * tile counts, is copied from `order_cache` when an earlier plan of this shape had tile
 * counts with the same 64-bit hash, and otherwise ranked as in sinkattn_block_sparse_plan
 * and then stored in the cache (round robin over `cache_entries` entries).  Results equal
 * sinkattn_block_sparse_plan's; a hash collision could only give a valid but less balanced
 * launch order (every order of a shape lists the same q-blocks once each).
 * order_cache: int32 buffer of sinkattn_block_sparse_order_cache_ints(B, H, nqb, entries)
 * ints, zero-filled before its first use, kept for one shape (B, H, nqb) and used by calls
 * ordered on one stream (calls that share a cache concurrently race); 1 <= entries <= 4096.
 * ---------------------------------------------------------------------------------- */
int64_t sinkattn_block_sparse_order_cache_ints(int64_t B, int64_t H, int64_t nqb,
                                               int64_t entries);
int sinkattn_block_sparse_plan_cached(const uint8_t* mask, const int64_t mask_strides[4],
                                      int64_t B, int64_t H, int64_t nqb, int64_t nkb,
                                      int32_t* counts, int32_t* idx, int32_t* order,
                                      int32_t* order_cache, int64_t cache_entries,
                                      void* stream);

/* ------------------------------------------------------------------------------------
 * Block-sparse flash-attention forward, 128x128 tiles.
 *
 * Replaces `block_sparse_attn_func` as called by `_block_sparse_attn`
 * (sinkattention/sparse_attention.py:710-776): for every query row of q-block qb the
 * keys of the listed key blocks (and only keys < Nk) are attended:
 *     out = softmax(scale * Q K^T + M) V,   lse = log(sum(exp(scale * Q K^T + M)))
 * with M = 0 on listed tiles and -inf elsewhere.  q/k/v/out are BHSD-addressed (see
 * above), dtype one of sinkattn_dtype (f32 operands are rounded to bf16 for the matrix
 * cores; accumulation and softmax are fp32).  lse is fp32 [B,H,Nq] contiguous, or NULL;
 * for D = 128 with 16-bit operands the row sums add the 16-bit P values the PV product uses,
 * so lse is within log(1 + 2^-8) of the exact value (bf16; 2^-11 for f16).
 * A row with no listed key block gets out = 0 and lse = +inf.
 * counts/idx/order come from sinkattn_block_sparse_plan (order may be NULL: one
 * work-group per row in row order).
 * D must be 32, 64 or 128 (the head dims of the external kernel the reference calls).
 * ---------------------------------------------------------------------------------- */
int sinkattn_block_sparse_fwd(const void* q, const void* k, const void* v, int dtype,
                              int64_t B, int64_t H, int64_t Nq, int64_t Nk, int64_t D,
                              const int64_t q_strides[4], const int64_t k_strides[4],
                              const int64_t v_strides[4],
                              void* out, const int64_t out_strides[4], float* lse,
                              const int32_t* counts, const int32_t* idx,
                              const int32_t* order, int64_t nqb, int64_t nkb,
                              float softmax_scale, void* stream);

/* ------------------------------------------------------------------------------------
 * Block-sparse forward fused with the compensation branch ("pooled_kv" dynamic mode with
 * adaptive mixing).
 *
 * Replaces the sparse call, the attention over the pooled K/V and `_mix_attention_outputs`
 * of `WanSinkSparseInnerAttention.forward` (wanx/runtime/sink_sparse_wan.py:194-265;
 * sinkattention/sparse_attention.py:898-919) and of the Z-Image image rows
 * (zimg/runtime/sink_sparse_zimage.py:553-592).  The reference computes
 *     out = a*out_s + (1-a)*out_d,  a = exp(lse_s) / (exp(lse_s) + gap*exp(lse_d)),
 * which equals attention over the listed keys plus every pooled key counted `gap`
 * times.  Here the q-blocks qb < comp_qblocks attend, after their listed tiles, every
 * key of kd/vd [B,H,Nd,D] (BHSD-addressed, row strides equal to k's/v's) with log_gap =
 * ln(gap) added to the scaled logits, in one online softmax; other q-blocks are plain
 * block-sparse rows.  lse (optional) is the LSE of that union.  bf16/f16, D = 128.
 * ---------------------------------------------------------------------------------- */
int sinkattn_block_sparse_fwd_comp(const void* q, const void* k, const void* v, int dtype,
                                   int64_t B, int64_t H, int64_t Nq, int64_t Nk, int64_t D,
                                   const int64_t q_strides[4], const int64_t k_strides[4],
                                   const int64_t v_strides[4],
                                   const void* kd, const void* vd,
                                   const int64_t kd_strides[4], const int64_t vd_strides[4],
                                   int64_t Nd, int64_t comp_qblocks, float log_gap,
                                   void* out, const int64_t out_strides[4], float* lse,
                                   const int32_t* counts, const int32_t* idx,
                                   const int32_t* order, int64_t nqb, int64_t nkb,
                                   float softmax_scale, void* stream);

/* ------------------------------------------------------------------------------------
 * Token mean pooling of the compensation branch.
 *
 * Replaces `_mean_pool_sequence_preserve_prefix` / `_mean_pool_sequence` /
 * `_pad_to_multiple` (sinkattention/sparse_attention.py:79-115): rows [0, prefix) of x
 * are copied; the remaining rows are averaged in groups of `gap` (a short last group
 * repeats row N-1, i.e. replicate padding).  fp32 sums, times fp32(1/gap), one rounding
 * to the dtype.  gap == 1 or prefix >= N copy x.  out has
 * sinkattn_mean_pool_tokens_rows(N, prefix, gap) rows.  D*elem_size must be a power of
 * two between 16 and 4096 bytes.
 * ---------------------------------------------------------------------------------- */
int64_t sinkattn_mean_pool_tokens_rows(int64_t N, int64_t prefix, int64_t gap);
int sinkattn_mean_pool_tokens(const void* x, int dtype, int64_t B, int64_t H, int64_t N,
                              int64_t D, const int64_t x_strides[4], int64_t prefix,
                              int64_t gap, void* out, const int64_t out_strides[4],
                              void* stream);

/* ------------------------------------------------------------------------------------
 * QK-norm + rotary embedding of Q and K in one pass.
 *
 * Replaces `apply_fast_qk_norm` + `apply_fast_rotary_qk` (wanx/runtime/fast_misc.py:
 * 216-234,834-864; their Triton kernels :308-340 and :432-500) and the norm + rotary of
 * `prepare_zimage_attention_tensors` (zimg/runtime/modify_zimage.py:8-43).  For each of
 * `rows` rows of C channels (row r at in + r*in_row_stride):
 *     rstd = 1/sqrt(sum(x^2)/C + eps);  y = dtype(x * rstd * w)        (w fp32 [C])
 *     then every channel pair (2i, 2i+1) of every D-channel head is rotated by the table
 *     row t = (r / rows_per_pos) % freq_rows:  (y0*re[t,i] - y1*im[t,i], y0*im[t,i] + y1*re[t,i])
 * freq_real/freq_imag fp32 [freq_rows, D/2] (both NULL: no rotation).  Wan: rows = B*N,
 * C = H*D, rows_per_pos = 1, freq_rows = N.  Z-Image: rows = B*N*H, C = D,
 * rows_per_pos = H, freq_rows = B*N.  Outputs written with out_row_stride; in-place is
 * allowed.  C <= 8192 (16-bit) / 4096 (f32) elements; D a multiple of 16 bytes.
 * ---------------------------------------------------------------------------------- */
int sinkattn_qk_norm_rotary(const void* q_in, const void* k_in, int dtype, int64_t rows,
                            int64_t C, int64_t D, int64_t in_row_stride,
                            const float* wq, const float* wk, float eps_q, float eps_k,
                            const float* freq_real, const float* freq_imag,
                            int64_t rows_per_pos, int64_t freq_rows,
                            void* q_out, void* k_out, int64_t out_row_stride, void* stream);

/* ------------------------------------------------------------------------------------
 * LSE mix of two attention outputs.
 *
 * Replaces `_mix_attention_outputs` (sinkattention/sparse_attention.py:898-919) for
 * callers that run the two branches separately, with the reference's rounding: each of
 * its torch ops on q.dtype tensors is one fp32 operation rounded to the dtype:
 *     wd = dyn_lse + log_gap; mx = max(sink_lse, wd); es = exp(sink_lse - mx);
 *     ed = exp(wd - mx); a = es / (es + ed); out = sink*a + dyn*(1 - a)
 * log_gap is the caller's q.dtype value of log(gap).  Outputs/inputs BHSD-addressed
 * [B,H,N,D]; the LSEs are [B,H,N] addressed by 3 strides, same dtype as the outputs.
 * ---------------------------------------------------------------------------------- */
int sinkattn_lse_mix(const void* sink_out, const int64_t sink_strides[4],
                     const void* sink_lse, const int64_t sink_lse_strides[3],
                     const void* dyn_out, const int64_t dyn_strides[4],
                     const void* dyn_lse, const int64_t dyn_lse_strides[3], int dtype,
                     int64_t B, int64_t H, int64_t N, int64_t D, float log_gap,
                     void* out, const int64_t out_strides[4], void* stream);

/* ------------------------------------------------------------------------------------
 * Exact block-mass pooling ("exact" pooling mode).
 *
 * Replaces `_compute_exact_block_mass_scores` (sinkattention/sparse_attention.py:145-227):
 *     P = softmax_rows(scale * Q K^T)                  (fp32, over all Nk keys)
 *     out[b,h,qb,kb] = mean over the rows r of q-block qb of  sum_{j in kb} P[r,j]
 * out is fp32 [B,H,nqb,nkb] contiguous, nqb = ceil(Nq/block), nkb = ceil(Nk/block).
 * block_size 16, 32, 64 or 128 with D 128: bf16/f16 inputs use the bf16/f16 matrix cores
 * (products are exact, sums fp32) and a device workspace of
 * sinkattn_block_mass_pool_workspace_bytes() bytes (per-row block sums of the resident
 * work-groups, queried for the current device); f32 inputs at block_size 128, D 128 use
 * the fp32 matrix cores (nkb <= 256) and need no workspace.  Every other shape
 * (block_size 1..1024, D 1..256, f32 otherwise) runs a generic kernel (fp32 dot products,
 * two passes over the keys, no workspace; the query may still return a size for a
 * matrix-core block size, which the call then leaves unused), limited by LDS to about
 * (160 KiB / 4 - 128 (D + 1) - 4160) key blocks.  Callers with a 16-bit head dim below 128
 * may zero-pad it to 128 to take the matrix cores (zeros leave every dot product exact).
 * ---------------------------------------------------------------------------------- */
size_t sinkattn_block_mass_pool_workspace_bytes(int64_t B, int64_t H, int64_t Nq, int64_t Nk,
                                                int64_t block_size, int dtype);
int sinkattn_block_mass_pool(const void* q, const void* k, int dtype,
                             int64_t B, int64_t H, int64_t Nq, int64_t Nk, int64_t D,
                             const int64_t q_strides[4], const int64_t k_strides[4],
                             int64_t block_size, float scale, float* out, void* workspace,
                             void* stream);

/* ------------------------------------------------------------------------------------
 * Row-normalised max-pool map ("triton" pooling mode).
 *
 * Replaces `attn_with_pooling` (sinkattention/pooling_kernel.py:194-248) minus its
 * all-zero `o` output and its [B,H,N,nd] scratch:
 *     R[r,kb]  = q.dtype( max_{j in kb} (q_r . k_j) * sm_scale * log2(e) )
 *     m_r      = max over kb of the unrounded block maxima
 *     Po[qb,kb]= q.dtype( max_{r in qb} exp2(R[r,kb] - m_r) )
 *     Po      /= q.dtype( sum_kb Po[qb,kb] )           (row normalisation in q.dtype)
 * Po is written in q.dtype (bf16, f16 or f32) as [B,H,nd,nd] contiguous.  kv head of query
 * head h is h / (H / Hk).  causal restricts row qb to kb <= qb and adds -1e6 to the
 * raw scores above the diagonal of the diagonal tile, as the reference does.  Keys and
 * rows >= N are excluded (the reference leaves ragged N undefined).  block_size in
 * {16, 32, 64, 128}, D in {16, 32, 64, 128, 256} (the reference's asserts).  bf16/f16 with
 * D 128 (nd <= 1024 at block_size 128) run the persistent MFMA kernel: `workspace` is a
 * device buffer of at least sinkattn_max_pool_workspace_bytes(...) bytes (per-(row,
 * key-block) maxima of the rows in flight); calls that share one workspace must be
 * ordered on one stream.  Other shapes run the generic kernel (no workspace; same LDS
 * bound as the generic block-mass kernel).
 * ---------------------------------------------------------------------------------- */
size_t sinkattn_max_pool_workspace_bytes(int64_t B, int64_t H, int64_t N, int64_t block_size,
                                         int dtype);
int sinkattn_max_pool(const void* q, const void* k, int dtype,
                      int64_t B, int64_t H, int64_t Hk, int64_t N, int64_t D,
                      const int64_t q_strides[4], const int64_t k_strides[4],
                      int64_t block_size, float sm_scale, int causal, void* po,
                      void* workspace, void* stream);

/* ------------------------------------------------------------------------------------
 * Mean-pooled block scores ("mean" pooling mode).
 *
 * Replaces `_compute_pooled_qk_block_scores`'s fallback branch with `_mean_pool_sequence`
 * / `_pad_to_multiple` (sinkattention/sparse_attention.py:79-94,138-142):
 *     Qp = mean over each block of rows of Q padded to a multiple of block by repeating
 *          its last row (likewise Kp);   out = softmax_rows(scale * Qp Kp^T)
 * out fp32 [B,H,nqb,nkb] contiguous.  workspace: sinkattn_mean_pool_workspace_bytes().
 * ---------------------------------------------------------------------------------- */
size_t sinkattn_mean_pool_workspace_bytes(int64_t B, int64_t H, int64_t Nq, int64_t Nk,
                                          int64_t D, int64_t block_size);
int sinkattn_mean_pool_scores(const void* q, const void* k, int dtype,
                              int64_t B, int64_t H, int64_t Nq, int64_t Nk, int64_t D,
                              const int64_t q_strides[4], const int64_t k_strides[4],
                              int64_t block_size, float scale, void* workspace,
                              float* out, void* stream);

/* ------------------------------------------------------------------------------------
 * Direct-mean coverage mask.
 *
 * Replaces `_build_direct_mean_coverage_mask` + `_build_offline_required_mask`
 * (sinkattention/sparse_attention.py:241-376), bit-exact with the reference's CPU torch
 * arithmetic.  scores: fp32 [H,nq,nk] contiguous.  Required blocks: every row's first
 * `req_k` columns and the first `req_q` rows entirely (both 0 when the reference's
 * required mask is None).  mode 0 = "joint" branch, 1 = "video_residual" branch with
 * `text_blocks` leading text blocks.  coverage is the already-clamped fp32 value.
 * Outputs: mask uint8 [H,nq,nk]; counts int32 [H,nq]; idx int32 [H,nq,nk] (ascending
 * key blocks of each row, counts[r] valid entries).  counts/idx may be NULL.
 * The reference's empty-row fallback is reproduced as written: if any row of the whole
 * tensor ends up empty, every row r gets mask[r, top1(r)] = (row r was empty), which
 * also clears that bit in non-empty rows.  workspace: *_workspace_bytes(H, nq).
 * nk <= 4096.
 * ---------------------------------------------------------------------------------- */
size_t sinkattn_coverage_mask_workspace_bytes(int64_t H, int64_t nq);
int sinkattn_coverage_mask(const float* scores, int64_t H, int64_t nq, int64_t nk,
                           float coverage, int keep_diagonal, int64_t req_q,
                           int64_t req_k, int mode, int64_t text_blocks,
                           uint8_t* mask, int32_t* counts, int32_t* idx,
                           void* workspace, void* stream);

/* ------------------------------------------------------------------------------------
 * Block-sparse forward from a bool mask, allocating nothing.
 *
 * No counterpart in the reference.  It is for callers that cannot allocate device memory:
 * code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * Same as sinkattn_block_sparse_plan followed by sinkattn_block_sparse_fwd (same checks,
 * kernels and results), but the plan (counts, index lists, launch order) is kept in a
 * static device array of SINKATTN_NOALLOC_SCRATCH_BYTES that the library owns, one per GPU,
 * held until the process ends.  The caller passes the mask (uint8/bool
 * [B,H,ceil(Nq/128),ceil(Nk/128)] with element strides, as for the plan) and the inputs and
 * outputs (as for the forward).  No device memory is allocated or freed.
 * Limit: 4 bytes per row for the counts, 4 per launch slot, and 4 * nkb per row for the
 * lists must fit the 32 MiB array: about 8 million mask entries B*H*nqb*nkb (Wan config 2
 * needs 1.6 million).  Larger calls return an invalid-argument status.
 * The array keeps the last call's plan and is shared by all calls on one GPU: calls on one
 * stream are ordered, but calls that overlap on one GPU (several streams or threads at
 * once) race and must not be issued.  The array is part of the library's code object, so
 * every GPU that loads the library reserves its 32 MiB, whether or not this function is
 * called.  The first call on each GPU looks up the array's device address and must not run
 * under stream capture (it returns an invalid-argument status there): make one call outside
 * capture first; later calls may be captured into a graph.
 * ---------------------------------------------------------------------------------- */
#define SINKATTN_NOALLOC_SCRATCH_BYTES (32u << 20)
int sinkattn_block_sparse_attn_noalloc(const uint8_t* mask, const int64_t mask_strides[4],
                                       const void* q, const void* k, const void* v, int dtype,
                                       int64_t B, int64_t H, int64_t Nq, int64_t Nk, int64_t D,
                                       const int64_t q_strides[4], const int64_t k_strides[4],
                                       const int64_t v_strides[4], void* out,
                                       const int64_t out_strides[4], float* lse,
                                       float softmax_scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SINKATTN_H_ */
