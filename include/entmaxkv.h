/* EntmaxKV for AMD Instinct MI355X (gfx950): C ABI of the sparse-entmax paged
 * decode path.
 *
 * Every entry point takes raw device pointers, element strides and a
 * hipStream_t passed as void*.  Nothing here allocates device memory:
 * workspaces are caller-owned and sized by the *_workspace_bytes queries;
 * they need no initialisation.  Calls that share a workspace must not run
 * concurrently.  Return value: 0 on success, EKV_ERR_ARG (-1) for a rejected
 * argument (nothing launched), EKV_ERR_HIP (-2) for a launch failure; the
 * message is in ekv_last_error() (thread-local).
 *
 * Ragged batches: entry points with a `seq_lens` argument accept per-sequence
 * lengths [B] (int32, device).  Sequence b then uses its own page count,
 * last page and statistics length; the scalar sizes (seq_len, num_pages,
 * pages_for_stats, ...) describe the longest sequence and fix the strides.
 * Null keeps one length for the whole batch.  This has no counterpart in the
 * reference, whose cache holds one length (kv_cache.py:23-38).
 *
 * dtype codes: 0 = fp32, 1 = fp16, 2 = bf16 (storage type of q/K/V/stats).
 * Head dim D: D / (16 / sizeof(dtype)) must be a power of two in [4, 64]
 * (fp16/bf16: 32..512, fp32: 16..256).  GQA group H / Hkv in {1, 2, 4, 8}.
 * Reference paths below are relative to the deep-spin/entmaxkv repository.
 */
#ifndef ENTMAXKV_H
#define ENTMAXKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EKV_ABI_VERSION 5

const char* ekv_last_error(void);
int ekv_abi_version(void);
/* Source hash of this build: the first 16 hex digits of a SHA-256 over the
 * library's sources, this header and the compile flags (written by the build
 * script).  Profiles record it, so that a measurement can be tied to the
 * library that produced it.  No counterpart in the reference. */
const char* ekv_build_id(void);

/* Per-page key statistics over pages [page_begin, page_end): min, max, mean and
 * population std (clamped >= 1e-6) of rows [p*ps, min((p+1)*ps, seq_len)).
 * Replaces the page loop of PagedKVCache.initialize, kv_cache.py:40-70. */
int ekv_page_stats(const void* k, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_row,
                   void* kmin, void* kmax, void* kmean, void* kstd, int64_t s_stride_b,
                   int64_t s_stride_h, int64_t s_stride_page, int B, int Hkv, int D, int seq_len,
                   const int32_t* seq_lens, int page_size, int page_begin, int page_end,
                   int dtype, void* stream);

/* In-place append of one token per (b, kv head) at row `pos` (or
 * pos_per_batch[b] when non-null, negative = skip) and recompute of that
 * page's statistics.  K and V share strides.  With block_table non-null
 * (see ekv_paged_entmax_decode) the row goes to block
 * block_table[b][pos / page_size] of the pool (skipped when the id lies
 * outside [0, bt_blocks)).  Replaces the torch.cat append
 * and last-page recompute of PagedKVCache.append, kv_cache.py:72-116. */
int ekv_append(const void* k_new, const void* v_new, int64_t new_stride_b, int64_t new_stride_h,
               void* k, void* v, int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_row,
               void* kmin, void* kmax, void* kmean, void* kstd, int64_t s_stride_b,
               int64_t s_stride_h, int64_t s_stride_page, int B, int Hkv, int D, int pos,
               const int32_t* pos_per_batch, const int32_t* block_table, int64_t bt_stride_b,
               int bt_blocks, int page_size, int dtype, void* stream);

/* Page criticality scores [B, H, num_pages] (query dtype, contiguous):
 * sum_d max(q_d kmin_pd, q_d kmax_pd) (+ ALiBi bonus when alibi_slopes [H] is
 * non-null).  Replaces triton_estimate_page_criticality,
 * kernels/page_criticality.py:107-187.  When k_select >= 0 the top-k page
 * table of ekv_topk_pages is produced by the same call. */
int ekv_page_criticality(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kmin,
                         const void* kmax, int64_t s_stride_b, int64_t s_stride_h,
                         int64_t s_stride_page, const float* alibi_slopes, void* scores, int B,
                         int H, int Hkv, int D, int num_pages, int page_size, int seq_len,
                         int q_pos, int k_select, int last_page, const int32_t* seq_lens,
                         int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h,
                         int dtype, void* stream);

/* Top-k page table per (b, kv head): the k pages with the largest score (group
 * maximum under GQA), ascending, ties to the lower index, then `last_page`
 * at slot k when last_page >= 0.  Replaces torch.topk + the index buffer of
 * attention_topk.py:52-71 and kv_cache.py:167-185. */
int ekv_topk_pages(const void* scores, int B, int H, int Hkv, int num_pages, int k, int last_page,
                   int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h, int dtype,
                   void* stream);

/* Workspace for ekv_paged_entmax_decode, ekv_topk_paged_entmax_decode and
 * ekv_gaussian_paged_entmax_decode: fp32 score rows, then one 8-byte word
 * per (b, head) for the paired launches.  Any contents on entry. */
int64_t ekv_decode_workspace_bytes(int B, int H, int Hkv, int D, int splits, int max_tokens);

/* Paged alpha-entmax decode over the compacted page table (keyed by kv head).
 * tau_mode 0: exact (histogram init + `iters` bracketed Halley steps), the
 *   final tau is written to tau [B, H];
 * tau_mode 1: tau_in [B, H] holds the starting value; `iters` unbounded
 *   Halley/Newton corrections, final tau written to tau (may alias tau_in).
 * qscale = (alpha-1)/sqrt(D) rounded to the storage dtype.  kv_rows bounds
 * the rows addressable per (b, kv head); out-of-range page ids are skipped.
 * K/V addressing: with block_table null, row r of (b, kv head) is at
 * b * kv_stride_b + kv_head * kv_stride_h + r * kv_stride_row (the
 * reference's contiguous cache); with a block table [B, >= kv_rows /
 * page_size] int32 (row stride bt_stride_b) over a pool of bt_blocks blocks,
 * it is at blk * kv_stride_b + kv_head * kv_stride_h + (r % page_size) *
 * kv_stride_row with blk = block_table[b][r / page_size] (e.g. a pool
 * [bt_blocks, Hkv, page_size, D]); block ids outside [0, bt_blocks) are
 * skipped.  The block table has no counterpart in the reference, whose cache
 * is contiguous (kv_cache.py:81-82).  kv_stride_b and kv_stride_h must be
 * multiples of kv_stride_row.
 * Replaces kernels/adadecode_paged.py:567-762 and
 * kernels/adadecode_paged_gaussian_tau.py:192-331. */
int ekv_paged_entmax_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k,
                            const void* v, int64_t kv_stride_b, int64_t kv_stride_h,
                            int64_t kv_stride_row, int64_t kv_rows, const int32_t* block_table,
                            int64_t bt_stride_b, int bt_blocks, const int32_t* page_indices,
                            int64_t pi_stride_b, int64_t pi_stride_h, int n_slots,
                            const int32_t* cache_seqlens, int64_t cs_stride_b, int64_t cs_stride_h,
                            const int32_t* q_seqlens, const float* alibi_slopes,
                            const float* tau_in, float* tau, int tau_mode, int iters, void* out, int64_t out_stride_b,
                            int64_t out_stride_h, float alpha, float qscale, int page_size, int B,
                            int H, int Hkv, int D, int splits, int max_tokens, void* workspace,
                            int64_t workspace_bytes, int dtype, void* stream);

/* One top-k decode step: criticality scores of pages [0, num_pages), the
 * top-k page table (+ last_page at slot k) written to page_indices, then the
 * exact-tau decode (tau_mode 0 of ekv_paged_entmax_decode, `niter` Halley
 * steps) over the selected pages, tau to tau [B, H].  Arguments mean what they
 * mean in ekv_page_criticality and ekv_paged_entmax_decode; ALiBi slopes serve
 * both.  When every (b, kv head) fits one workgroup with its keys, page table
 * and scores in LDS this is a single launch, otherwise the two calls above.
 * Replaces the selection + decode sequence of sparse_attention_decode_paged,
 * attention_topk.py:45-98. */
int ekv_topk_paged_entmax_decode(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kmin, const void* kmax,
    int64_t s_stride_b, int64_t s_stride_h, int64_t s_stride_page, void* scores, int num_pages,
    int seq_len, int q_pos, int k_select, int last_page, const void* k, const void* v,
    int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_row, int64_t kv_rows,
    const int32_t* block_table, int64_t bt_stride_b, int bt_blocks,
    int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h,
    const int32_t* cache_seqlens, int64_t cs_stride_b, int64_t cs_stride_h,
    const int32_t* q_seqlens, const float* alibi_slopes, const int32_t* seq_lens, float* tau,
    int niter, void* out, int64_t out_stride_b, int64_t out_stride_h, float alpha, float qscale,
    int page_size, int B, int H, int Hkv, int D, int splits, int max_tokens, void* workspace,
    int64_t workspace_bytes, int dtype, void* stream);

/* ekv_append followed by ekv_topk_paged_entmax_decode, the step of
 * sparse_attention_decode_paged with append_cache=True (attention_topk.py:
 * 45-47 then 52-98, kv_cache.py:72-116): row `pos` of K and V comes from
 * k_new / v_new [B, Hkv, D] (row strides new_stride_b, new_stride_h) and the
 * statistics of page pos / page_size are recomputed (kmean, kstd with the
 * strides of kmin, kmax).  seq_len, q_pos, cache_seqlens and kv_rows already
 * count the new row.  Uniform batches only (seq_lens null).  In the fused
 * launch the append runs inside the top-k kernel (its page is the last one,
 * which the criticality scan never reads), else as its own launch first. */
int ekv_append_topk_paged_entmax_decode(
    const void* k_new, const void* v_new, int64_t new_stride_b, int64_t new_stride_h,
    void* kmean, void* kstd, int pos,
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kmin, const void* kmax,
    int64_t s_stride_b, int64_t s_stride_h, int64_t s_stride_page, void* scores, int num_pages,
    int seq_len, int q_pos, int k_select, int last_page, const void* k, const void* v,
    int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_row, int64_t kv_rows,
    const int32_t* block_table, int64_t bt_stride_b, int bt_blocks,
    int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h,
    const int32_t* cache_seqlens, int64_t cs_stride_b, int64_t cs_stride_h,
    const int32_t* q_seqlens, const float* alibi_slopes, const int32_t* seq_lens, float* tau,
    int niter, void* out, int64_t out_stride_b, int64_t out_stride_h, float alpha, float qscale,
    int page_size, int B, int H, int Hkv, int D, int splits, int max_tokens, void* workspace,
    int64_t workspace_bytes, int dtype, void* stream);

/* Size of the static device scratch of ekv_topk_paged_entmax_decode_noalloc. */
#define EKV_NOALLOC_SCRATCH_BYTES (16ll << 20)

/* ekv_topk_paged_entmax_decode without the workspace arguments: it calls no
 * allocator.  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under hipGraph capture, serving loops that
 * forbid hipMalloc).  The workspace is a static device array of
 * EKV_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; a step
 * whose workspace (ekv_decode_workspace_bytes: B * H * max_tokens * 4 bytes
 * of scores plus B * H * 8 bytes of pair words, each rounded up to 256) exceeds it is rejected with EKV_ERR_ARG and nothing is launched.  Every
 * call on one GPU shares that GPU's array, so calls that overlap on one GPU
 * (other streams, other host threads) race and must be serialised by the
 * caller.  Results equal ekv_topk_paged_entmax_decode's. */
int ekv_topk_paged_entmax_decode_noalloc(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kmin, const void* kmax,
    int64_t s_stride_b, int64_t s_stride_h, int64_t s_stride_page, void* scores, int num_pages,
    int seq_len, int q_pos, int k_select, int last_page, const void* k, const void* v,
    int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_row, int64_t kv_rows,
    const int32_t* block_table, int64_t bt_stride_b, int bt_blocks,
    int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h,
    const int32_t* cache_seqlens, int64_t cs_stride_b, int64_t cs_stride_h,
    const int32_t* q_seqlens, const float* alibi_slopes, const int32_t* seq_lens, float* tau,
    int niter, void* out, int64_t out_stride_b, int64_t out_stride_h, float alpha, float qscale,
    int page_size, int B, int H, int Hkv, int D, int splits, int max_tokens, int dtype,
    void* stream);

/* Workspace for ekv_gaussian_moments / ekv_gaussian_page_stats (the partial
 * sums of the global moments; needs no initialisation). */
int64_t ekv_gaussian_workspace_bytes(int B, int H, int Hkv, int D, int pages, int dtype);

/* Per-page score moments mu_p, sigma_p [B, H, pages_for_stats] (fp32, mu_p
 * with the ALiBi page-mean bias when alibi_slopes is non-null) and, in the
 * workspace, each workgroup's partial sums of the global moments: the first
 * launch of ekv_gaussian_page_stats and of the fused Gaussian step.  The
 * number of partials per head depends on whether seq_lens is given, so the
 * decode call that reads this workspace must be given the same seq_lens
 * (null or not).  Replaces the moment kernel of compute_page_gaussian_stats_triton
 * (kernels/gaussian_page_stats.py:8-121, 128-233). */
int ekv_gaussian_moments(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kmean,
                         const void* kstd, int64_t s_stride_b, int64_t s_stride_h,
                         int64_t s_stride_page, int pages_for_stats, const float* alibi_slopes,
                         int page_size, int seq_len, int n_tokens, const int32_t* seq_lens,
                         float* mu_p, float* sigma_p, int B, int H, int Hkv, int D,
                         void* workspace, int64_t workspace_bytes, int dtype, void* stream);

/* Per-page score moments mu_p, sigma_p [B, H, pages_for_stats] (fp32; mu_p
 * includes the ALiBi page-mean bias when alibi_slopes is non-null), per-head
 * mu_g, sigma_g, mean_var, var_means [B, H], and, when tau_hat is non-null,
 * the single-Gaussian tau-hat with n = n_tokens.  Replaces
 * compute_page_gaussian_stats_triton (kernels/gaussian_page_stats.py:128-233)
 * and gaussian_utils.py:130-181. */
int ekv_gaussian_page_stats(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                            const void* kmean, const void* kstd, int64_t s_stride_b,
                            int64_t s_stride_h, int64_t s_stride_page, int pages_for_stats,
                            const float* alibi_slopes, int page_size, int seq_len, float* mu_p,
                            float* sigma_p, float* mu_g, float* sigma_g, float* mean_var,
                            float* var_means, float* tau_hat, float alpha, int n_tokens,
                            int tau_iters, float tol, const int32_t* seq_lens, int B, int H,
                            int Hkv, int D, void* workspace, int64_t workspace_bytes, int dtype,
                            void* stream);

/* tau-hat for `count` independent single-Gaussian problems.  Replaces
 * solve_for_tau_hat_single_gaussian_gpu, kernels/tau_solver_gpu.py:128-158. */
int ekv_tau_single_gaussian(const float* mu_g, const float* sigma_g, float* tau_out, int count,
                            int n_tokens, float alpha, int iterations, float tol, void* stream);

/* Page-mixture tau-hat per row of [rows, pages] (uniform page count).
 * With seq_lens (ragged batch), row r mixes the statistics pages of sequence
 * r / rows_per_seq only.  Replaces
 * solve_for_tau_hat_page_gaussian_mixture_triton,
 * kernels/tau_mixture_solver_triton.py:172-240. */
int ekv_tau_page_mixture(const float* mu_p, const float* sigma_p, float* tau_out, int rows,
                         int pages, float page_count, float alpha, int max_iter, float tol,
                         const int32_t* seq_lens, int rows_per_seq, int page_size,
                         void* stream);

/* Threshold selection + ascending pack + last-page sentinel per (b, kv head),
 * tau floor per head, and (optional, fused) compacted cache lengths and tau
 * clamp.  auto_margins != 0 derives safety_margin_z and the page quantile from
 * the mean sigma_g on device (z_page_low/high are the page quantile z-values
 * for max_quantile 0.99/0.995).  Replaces select_gaussian_threshold_pack_triton
 * (kernels/selection_pack.py:201-272), gaussian_utils.py:163-169,
 * clamp_tau_to_selected_page_statistics_triton (kernels/tau_clamp.py:76-151)
 * and cache_seqlens_from_page_counts_triton (kernels/selection_pack.py:23-43). */
int ekv_select_gaussian_pack(const float* mu_p, const float* sigma_p, const float* tau_hat,
                             const float* sigma_g, int B, int H, int Hkv, int pages_for_stats,
                             int num_pages, float alpha, int auto_margins, float safety_margin_z,
                             float z_page, float z_page_low, float z_page_high,
                             float threshold_excess_margin_fraction, int32_t* page_indices,
                             int64_t pi_stride_b, int64_t pi_stride_h, int32_t* counts,
                             float* tau_floor, int32_t* cache_seqlens, int page_size,
                             int last_page_size, float* tau_clamped, float z_clamp, float eps,
                             float* effective_margins, const int32_t* seq_lens, void* stream);

/* One Gaussian-aware decode step after ekv_gaussian_moments (whose workspace
 * and mu_p / sigma_p it reads): global moments and tau-hat per head (unless
 * tau_hat_given, e.g. the page-mixture tau-hat under ALiBi), then the
 * selection of ekv_select_gaussian_pack (tau_clamped null = no clamp), then
 * the decode of ekv_paged_entmax_decode over the selected pages: tau_mode 1
 * starts from the clamped tau (or tau-hat) with `iters` corrections, tau_mode
 * 0 solves tau exactly with `iters` Halley steps.  The page table has
 * num_pages slots; max_tokens >= num_pages * page_size sizes the decode
 * workspace.  One launch per step when batch * kv heads fills the GPU,
 * otherwise the separate launches.  Replaces the selection + decode sequence
 * of sparse_attention_decode_gaussian_aware_entmax (attention_gaussian.py:
 * 68-122) with kernels/selection_pack.py:201-272, kernels/tau_clamp.py:76-151
 * and kernels/adadecode_paged_gaussian_tau.py:192-331. */
int ekv_gaussian_paged_entmax_decode(
    const void* moments_workspace, int64_t moments_workspace_bytes, const float* mu_p,
    const float* sigma_p, int pages_for_stats, int num_pages, float* mu_g, float* sigma_g,
    float* mean_var, float* var_means, float* tau_hat, int tau_hat_given, int n_tokens,
    int tau_iters, float tol, int auto_margins, float safety_margin_z, float z_page,
    float z_page_low, float z_page_high, float threshold_excess_margin_fraction,
    int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h, int32_t* counts,
    float* tau_floor, int32_t* cache_seqlens, int last_page_size, float* tau_clamped,
    float z_clamp, float eps, float* effective_margins, const void* q, int64_t q_stride_b,
    int64_t q_stride_h, const void* k, const void* v, int64_t kv_stride_b, int64_t kv_stride_h,
    int64_t kv_stride_row, int64_t kv_rows, const int32_t* block_table, int64_t bt_stride_b,
    int bt_blocks, const int32_t* q_seqlens, const float* alibi_slopes,
    const int32_t* seq_lens, float* tau, int tau_mode, int iters, void* out,
    int64_t out_stride_b, int64_t out_stride_h, float alpha, float qscale, int page_size, int B,
    int H, int Hkv, int D, int max_tokens, void* workspace, int64_t workspace_bytes, int dtype,
    void* stream);

/* Standalone tau clamp over a page list (kernels/tau_clamp.py:8-73). */
int ekv_tau_clamp(const float* tau, const float* mu_p, const float* sigma_p,
                  const int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h,
                  int n_slots, const int32_t* num_selected, int64_t ns_stride_b,
                  int64_t ns_stride_h, const float* tau_floor, float* out, int B, int H, int Hsel,
                  int pages_for_stats, float alpha, float z_clamp, float eps, void* stream);

/* max(count - 1, 0) * page_size + last_page_size (kernels/selection_pack.py:7-20). */
int ekv_cache_seqlens_from_counts(const int32_t* counts, int32_t* cache_seqlens, int n,
                                  int page_size, int last_page_size, void* stream);

/* Dense (non-paged) decode: one query token per head over a contiguous cache
 * k/v [B, Hkv, kv_rows, D] (row stride kv_stride_row, last dim contiguous),
 * exact tau (histogram init + `iters` bracketed Halley steps, as tau_mode 0
 * of ekv_paged_entmax_decode); head b, h attends to its first
 * cache_seqlens[b] rows.  With alibi_slopes, key j of (b, kv head) sits at
 * token_positions[b * pos_stride_b + kvh * pos_stride_h + j] (null: at j) and
 * the query at q_seqlens[b] - 1 (null: cache_seqlens[b] - 1).  The final tau
 * goes to tau [B, H].  Workspace: ekv_dense_decode_workspace_bytes bytes, no
 * initialisation.  Replaces sparse_attention_decode_orchestrator
 * (kernels/adadecode.py:754-1016). */
int64_t ekv_dense_decode_workspace_bytes(int B, int H, int64_t kv_rows);
int ekv_dense_entmax_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                            const void* k, const void* v, int64_t kv_stride_b,
                            int64_t kv_stride_h, int64_t kv_stride_row, int64_t kv_rows,
                            const int32_t* cache_seqlens, const int32_t* token_positions,
                            int64_t pos_stride_b, int64_t pos_stride_h,
                            const int32_t* q_seqlens, const float* alibi_slopes, float* tau,
                            int iters, void* out, int64_t out_stride_b, int64_t out_stride_h,
                            float alpha, float qscale, int B, int H, int Hkv, int D,
                            void* workspace, int64_t workspace_bytes, int dtype, void* stream);

/* Row-wise alpha-entmax over the last dimension: y[r] = entmax_alpha(x[r]) for
 * `rows` rows of n elements (row strides in elements, elements contiguous),
 * tau solved exactly (alpha 2 and 1.5: support refinement to the closed-form
 * root; other alpha: bracketed Halley to fp32 resolution); tau_out [rows]
 * (optional) receives the threshold on the (alpha - 1) x scale.  Replaces
 * _fwd_entmax (kernels/triton_entmax.py:364-533). */
int ekv_entmax_rows_forward(const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride,
                            int64_t rows, int n, float alpha, float* tau_out, int dtype,
                            void* stream);

/* Gradient of row-wise alpha-entmax: u = y^(2 - alpha) on the support,
 * dx = u dy - (sum u dy / sum u) u.  Replaces _bwd_entmax
 * (kernels/triton_entmax.py:536-612). */
int ekv_entmax_rows_backward(const void* y, int64_t y_row_stride, const void* dy,
                             int64_t dy_row_stride, void* dx, int64_t dx_row_stride,
                             int64_t rows, int n, float alpha, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ENTMAXKV_H */
