// C entry points of the paged decode (exact / given tau), the fused top-k
// decode step and the fused Gaussian select + decode step.  The kernels and
// their per-(dtype, group) launchers live in decode_device.h /
// decode_launch.h; decode_inst.hip instantiates them.
#include <atomic>

#include "decode_device.h"
#include "../../include/entmaxkv.h"

using namespace ekv;
using namespace ekv::dec;

namespace {

// The block pool of a cache that is not contiguous per (b, kv head): see
// DecodeArgs::block_table.
struct KvBlocks {
  const int32_t* table = nullptr;
  int64_t stride_b = 0;
  int count = 0;
};

// Checks shared by the decode entry points on the K/V addressing: support
// rows are kept as offsets in rows of kv_stride_row elements, and a block
// table needs a pool.
int check_kv_layout(const char* what, int64_t kv_stride_b, int64_t kv_stride_h,
                    int64_t kv_stride_row, const KvBlocks& blocks) {
  EKV_REQUIRE(kv_stride_row > 0 && kv_stride_b % kv_stride_row == 0 &&
                  kv_stride_h % kv_stride_row == 0,
              "%s: K/V strides must be multiples of the row stride", what);
  EKV_REQUIRE(!blocks.table || (blocks.count > 0 && blocks.stride_b >= 0),
              "%s: a block table needs bt_blocks > 0", what);
  return EKV_OK;
}

template <typename F>
int dispatch_group(int G, F&& f) {
  switch (G) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    default: return set_error(EKV_ERR_ARG, "GQA group size %d unsupported (1, 2, 4 or 8)", G);
  }
}

DecodeArgs make_decode_args(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k, const void* v,
    int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_row, int64_t kv_rows,
    const int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h, int n_slots,
    const int32_t* cache_seqlens, int64_t cs_stride_b, int64_t cs_stride_h,
    const int32_t* q_seqlens, const float* alibi_slopes, const float* tau_in, float* tau,
    int tau_mode, int iters, void* out, int64_t out_stride_b, int64_t out_stride_h, float alpha,
    float qscale, int page_size, int H, int Hkv, int splits, int max_tokens, void* workspace,
    const KvBlocks& blocks = KvBlocks{}) {
  DecodeArgs a;
  a.block_table = blocks.table;
  a.btsb = blocks.stride_b;
  a.bt_blocks = blocks.count;
  a.q = q;
  a.qsb = q_stride_b;
  a.qsh = q_stride_h;
  a.k = k;
  a.v = v;
  a.ksb = kv_stride_b;
  a.ksh = kv_stride_h;
  a.ksr = kv_stride_row;
  a.row_limit = kv_rows;
  a.page_indices = page_indices;
  a.pisb = pi_stride_b;
  a.pish = pi_stride_h;
  a.n_slots = n_slots;
  a.cache_seqlens = cache_seqlens;
  a.csb = cs_stride_b;
  a.csh = cs_stride_h;
  a.q_seqlens = q_seqlens;
  a.slopes = alibi_slopes;
  a.tau = tau;
  a.tau_in = tau_in;
  a.tau_mode = tau_mode;
  a.iters = iters;
  a.out = out;
  a.osb = out_stride_b;
  a.osh = out_stride_h;
  a.alpha = alpha;
  a.qscale = qscale;
  a.page_size = page_size;
  a.H = H;
  a.Hkv = Hkv;
  a.splits = splits;
  a.max_tokens = max_tokens;
  a.ws_scores = (float*)workspace;
  return a;
}

// Workgroups per head of the split scoring launch: about 128 tokens each, at
// most 256 (the choice of kernels.choose_splits for the same width).
int splits_for(int max_tokens) {
  int s = (max_tokens + 127) / 128;
  return s < 1 ? 1 : (s > 256 ? 256 : s);
}

}  // namespace

extern "C" int64_t ekv_decode_workspace_bytes(int B, int H, int Hkv, int D, int splits,
                                              int max_tokens) {
  (void)Hkv;
  (void)D;
  (void)splits;
  // fp32 scores [B, H, max_tokens], then the paired Gaussian launch's words
  return ((int64_t)B * H * max_tokens * 4 + 255) / 256 * 256 +
         ((int64_t)B * H * 8 + 255) / 256 * 256;
}

// The decode launch(es); force_split spreads every head over many workgroups
// (ragged batches, whose heads differ widely in length).
static int paged_decode(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k, const void* v,
    int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_row, int64_t kv_rows,
    const int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h, int n_slots,
    const int32_t* cache_seqlens, int64_t cs_stride_b, int64_t cs_stride_h,
    const int32_t* q_seqlens, const float* alibi_slopes, const float* tau_in, float* tau,
    int tau_mode, int iters, void* out, int64_t out_stride_b, int64_t out_stride_h, float alpha,
    float qscale, int page_size, int B, int H, int Hkv, int D, int splits, int max_tokens,
    void* workspace, int64_t workspace_bytes, int dtype, void* stream, bool force_split,
    const int32_t* positions = nullptr, int64_t pos_stride_b = 0, int64_t pos_stride_h = 0,
    const KvBlocks& blocks = KvBlocks{}) {
  EKV_REQUIRE(q && k && v && page_indices && cache_seqlens && tau && out && workspace,
              "ekv_paged_entmax_decode: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "ekv_paged_entmax_decode: bad heads");
  EKV_REQUIRE(page_size > 0 && n_slots > 0 && splits > 0 && max_tokens > 0 && kv_rows > 0,
              "ekv_paged_entmax_decode: bad sizes");
  EKV_REQUIRE(tau_mode == 0 || tau_mode == 1, "ekv_paged_entmax_decode: tau_mode %d", tau_mode);
  EKV_REQUIRE(tau_mode == 0 || tau_in, "ekv_paged_entmax_decode: given-tau mode needs tau_in");
  EKV_REQUIRE(iters >= 0, "ekv_paged_entmax_decode: iters %d", iters);
  EKV_REQUIRE(alpha > 1.0f, "ekv_paged_entmax_decode: alpha must be > 1");
  EKV_REQUIRE(workspace_bytes >= ekv_decode_workspace_bytes(B, H, Hkv, D, splits, max_tokens),
              "ekv_paged_entmax_decode: workspace too small");
  if (int rc = check_kv_layout("ekv_paged_entmax_decode", kv_stride_b, kv_stride_h,
                               kv_stride_row, blocks))
    return rc;
  DecodeArgs a = make_decode_args(q, q_stride_b, q_stride_h, k, v, kv_stride_b, kv_stride_h,
                                  kv_stride_row, kv_rows, page_indices, pi_stride_b, pi_stride_h,
                                  n_slots, cache_seqlens, cs_stride_b, cs_stride_h, q_seqlens,
                                  alibi_slopes, tau_in, tau, tau_mode, iters, out, out_stride_b,
                                  out_stride_h, alpha, qscale, page_size, H, Hkv, splits,
                                  max_tokens, workspace, blocks);
  a.positions = positions;
  a.posb = pos_stride_b;
  a.posh = pos_stride_h;
  hipStream_t s = (hipStream_t)stream;
  const int G = H / Hkv;
  const bool head_path = one_workgroup_per_head(B * Hkv, force_split);
  const int cap = kStageBytes / 4 / (G > 0 ? G : 1);
  a.stage_cap = head_path ? (max_tokens < cap ? max_tokens : cap) : 0;
  a.scores_ready = head_path ? 0 : 1;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    return dispatch_group(G, [&](auto gv) {
      return dec::Launch<T, decltype(gv)::value>::decode(a, B, Hkv, D, head_path, s);
    });
  });
}

extern "C" int ekv_paged_entmax_decode(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k, const void* v,
    int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_row, int64_t kv_rows,
    const int32_t* block_table, int64_t bt_stride_b, int bt_blocks,
    const int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h, int n_slots,
    const int32_t* cache_seqlens, int64_t cs_stride_b, int64_t cs_stride_h,
    const int32_t* q_seqlens, const float* alibi_slopes, const float* tau_in, float* tau,
    int tau_mode, int iters, void* out, int64_t out_stride_b, int64_t out_stride_h, float alpha,
    float qscale, int page_size, int B, int H, int Hkv, int D, int splits, int max_tokens,
    void* workspace, int64_t workspace_bytes, int dtype, void* stream) {
  return paged_decode(q, q_stride_b, q_stride_h, k, v, kv_stride_b, kv_stride_h, kv_stride_row,
                      kv_rows, page_indices, pi_stride_b, pi_stride_h, n_slots, cache_seqlens,
                      cs_stride_b, cs_stride_h, q_seqlens, alibi_slopes, tau_in, tau, tau_mode,
                      iters, out, out_stride_b, out_stride_h, alpha, qscale, page_size, B, H, Hkv,
                      D, splits, max_tokens, workspace, workspace_bytes, dtype, stream, false,
                      nullptr, 0, 0, KvBlocks{block_table, bt_stride_b, bt_blocks});
}

// The appended row of ekv_append_topk_paged_entmax_decode (null: none).
struct AppendSpec {
  const void* k_new;
  const void* v_new;
  int64_t nsb, nsh;
  void* kmean;
  void* kstd;
  int pos;
};

static int topk_step(
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
    int64_t workspace_bytes, int dtype, void* stream,
    const AppendSpec* app) {
  const KvBlocks blocks{block_table, bt_stride_b, bt_blocks};
  EKV_REQUIRE(q && kmin && kmax && scores && k && v && page_indices && cache_seqlens && tau &&
                  out && workspace,
              "ekv_topk_paged_entmax_decode: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "ekv_topk_paged_entmax_decode: bad heads");
  EKV_REQUIRE(num_pages > 0 && k_select > 0 && k_select <= num_pages && page_size > 0,
              "ekv_topk_paged_entmax_decode: bad page selection (k %d of %d pages)", k_select,
              num_pages);
  EKV_REQUIRE(niter >= 0 && alpha > 1.0f && splits > 0 && max_tokens > 0 && kv_rows > 0,
              "ekv_topk_paged_entmax_decode: bad decode parameters");
  EKV_REQUIRE(workspace_bytes >= ekv_decode_workspace_bytes(B, H, Hkv, D, splits, max_tokens),
              "ekv_topk_paged_entmax_decode: workspace too small");
  if (int rc = check_kv_layout("ekv_topk_paged_entmax_decode", kv_stride_b, kv_stride_h,
                               kv_stride_row, blocks))
    return rc;
  const int n_slots = k_select + (last_page >= 0 ? 1 : 0);
  const int G = H / Hkv;
  // the standalone append launch, ahead of any launch that reads the cache
  auto append_first = [&]() {
    if (!app) return (int)EKV_OK;
    return ekv_append(app->k_new, app->v_new, app->nsb, app->nsh, const_cast<void*>(k),
                      const_cast<void*>(v), kv_stride_b, kv_stride_h, kv_stride_row,
                      const_cast<void*>(kmin), const_cast<void*>(kmax), app->kmean, app->kstd,
                      s_stride_b, s_stride_h, s_stride_page, B, Hkv, D, app->pos, nullptr,
                      block_table, bt_stride_b, bt_blocks, page_size, dtype, stream);
  };
  auto two_launches = [&]() {
    if (int rc = append_first()) return rc;
    int rc = ekv_page_criticality(q, q_stride_b, q_stride_h, kmin, kmax, s_stride_b, s_stride_h,
                                  s_stride_page, alibi_slopes, scores, B, H, Hkv, D, num_pages,
                                  page_size, seq_len, q_pos, k_select, last_page, seq_lens,
                                  page_indices, pi_stride_b, pi_stride_h, dtype, stream);
    if (rc) return rc;
    return paged_decode(q, q_stride_b, q_stride_h, k, v, kv_stride_b, kv_stride_h, kv_stride_row,
                        kv_rows, page_indices, pi_stride_b, pi_stride_h, n_slots, cache_seqlens,
                        cs_stride_b, cs_stride_h, q_seqlens, alibi_slopes, nullptr, tau, 0, niter,
                        out, out_stride_b, out_stride_h, alpha, qscale, page_size, B, H, Hkv, D,
                        splits, max_tokens, workspace, workspace_bytes, dtype, stream,
                        seq_lens != nullptr, nullptr, 0, 0, blocks);
  };
  // one launch when every head fills a workgroup and its keys, page table and
  // scores stay in LDS; otherwise criticality+top-k, then the decode
  if (!one_workgroup_per_head(B * Hkv, seq_lens != nullptr) || num_pages > topk::kMaxStagedKeys ||
      n_slots > kTablePages)
    return two_launches();
  const int tokens = max_tokens < n_slots * page_size ? max_tokens : n_slots * page_size;
  DecodeArgs a = make_decode_args(q, q_stride_b, q_stride_h, k, v, kv_stride_b, kv_stride_h,
                                  kv_stride_row, kv_rows, page_indices, pi_stride_b, pi_stride_h,
                                  n_slots, cache_seqlens, cs_stride_b, cs_stride_h, q_seqlens,
                                  alibi_slopes, nullptr, tau, 0, niter, out, out_stride_b,
                                  out_stride_h, alpha, qscale, page_size, H, Hkv, splits,
                                  max_tokens, workspace, blocks);
  a.stage_cap = tokens;
  a.scores_ready = 0;
  SelectArgs t;
  t.kmin = kmin;
  t.kmax = kmax;
  t.ssb = s_stride_b;
  t.ssh = s_stride_h;
  t.ssp = s_stride_page;
  t.scores = scores;
  t.num_pages = num_pages;
  t.seq_len = seq_len;
  t.q_pos = q_pos;
  t.k = k_select;
  t.last_page = last_page;
  t.key_cap = num_pages;
  t.seq_lens = seq_lens;
  t.prescored = 0;
  t.scan_rev = topk::next_scan_order();
  t.scan_nt = stream_nt(B, Hkv, num_pages, D, dtype) ? 1 : 0;
  if (app) {
    t.app_k = app->k_new;
    t.app_v = app->v_new;
    t.app_nsb = app->nsb;
    t.app_nsh = app->nsh;
    t.app_kmean = app->kmean;
    t.app_kstd = app->kstd;
    t.app_pos = app->pos;
  }
  hipStream_t s = (hipStream_t)stream;
  // fewer (b, kv head) pairs than CUs: the criticality scan, the step's
  // largest part, runs over every CU in a launch of its own, and the fused
  // launch starts from its scores
  if (G <= 2 && 2 * B * Hkv <= device_cus() && max_tokens >= 2 &&
      ((uintptr_t)workspace & 7) == 0) {
    // two workgroups per (b, kv head) share its scan inside the one launch;
    // their arrival words are the first B * Hkv 8-byte words of the
    // workspace, whose scores this launch does not use.  (Groups of 4 and 8
    // measured slower paired: config 4 102.9 against 108.6 us.)
    static std::atomic<unsigned long long> launches{0};
    t.pair_cnt = (unsigned long long*)workspace;
    t.pair_tag = ((launches.fetch_add(1, std::memory_order_relaxed) + 1) *
                  0x9E3779B97F4A7C15ull) | 1ull;
  } else if (B * Hkv < device_cus()) {
    const int rc = topk::criticality_split_scores(
        q, q_stride_b, q_stride_h, kmin, kmax, s_stride_b, s_stride_h, s_stride_page,
        alibi_slopes, scores, B, H, Hkv, D, num_pages, page_size, seq_len, q_pos, nullptr, dtype,
        s, t.scan_rev, t.scan_nt);
    if (rc) return rc;
    t.prescored = 1;
  }
  int handled = 0;
  auto fused = [&]() {
    return dispatch_dtype(dtype, [&](auto tv) {
      using T = decltype(tv);
      return dispatch_group(G, [&](auto gv) {
        return dec::Launch<T, decltype(gv)::value>::topk(a, t, B, Hkv, D, tokens, s, &handled);
      });
    });
  };
  int rc = fused();
  if (rc || handled) return rc;
  if (t.pair_cnt) {
    // the pairs do not fit (a group's keys not in LDS): the prescored launch
    t.pair_cnt = nullptr;
    rc = topk::criticality_split_scores(q, q_stride_b, q_stride_h, kmin, kmax, s_stride_b,
                                        s_stride_h, s_stride_page, alibi_slopes, scores, B, H,
                                        Hkv, D, num_pages, page_size, seq_len, q_pos, nullptr,
                                        dtype, s, t.scan_rev, t.scan_nt);
    if (rc) return rc;
    t.prescored = 1;
    rc = fused();
    if (rc || handled) return rc;
  }
  return two_launches();
}

extern "C" int ekv_topk_paged_entmax_decode(
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
    int64_t workspace_bytes, int dtype, void* stream) {
  return topk_step(q, q_stride_b, q_stride_h, kmin, kmax, s_stride_b, s_stride_h, s_stride_page,
                   scores, num_pages, seq_len, q_pos, k_select, last_page, k, v, kv_stride_b,
                   kv_stride_h, kv_stride_row, kv_rows, block_table, bt_stride_b, bt_blocks,
                   page_indices, pi_stride_b, pi_stride_h, cache_seqlens, cs_stride_b,
                   cs_stride_h, q_seqlens, alibi_slopes, seq_lens, tau, niter, out, out_stride_b,
                   out_stride_h, alpha, qscale, page_size, B, H, Hkv, D, splits, max_tokens,
                   workspace, workspace_bytes, dtype, stream, nullptr);
}

extern "C" int ekv_append_topk_paged_entmax_decode(
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
    int64_t workspace_bytes, int dtype, void* stream) {
  EKV_REQUIRE(k_new && v_new && kmean && kstd && pos >= 0 && !seq_lens,
              "ekv_append_topk_paged_entmax_decode: null pointer, negative position or ragged "
              "batch (use ekv_append first)");
  EKV_REQUIRE(pos < kv_rows, "ekv_append_topk_paged_entmax_decode: row %d beyond kv_rows", pos);
  const AppendSpec app{k_new, v_new, new_stride_b, new_stride_h, kmean, kstd, pos};
  return topk_step(q, q_stride_b, q_stride_h, kmin, kmax, s_stride_b, s_stride_h, s_stride_page,
                   scores, num_pages, seq_len, q_pos, k_select, last_page, k, v, kv_stride_b,
                   kv_stride_h, kv_stride_row, kv_rows, block_table, bt_stride_b, bt_blocks,
                   page_indices, pi_stride_b, pi_stride_h, cache_seqlens, cs_stride_b,
                   cs_stride_h, q_seqlens, alibi_slopes, seq_lens, tau, niter, out, out_stride_b,
                   out_stride_h, alpha, qscale, page_size, B, H, Hkv, D, splits, max_tokens,
                   workspace, workspace_bytes, dtype, stream, &app);
}

extern "C" int ekv_gaussian_paged_entmax_decode(
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
    void* stream) {
  const KvBlocks blocks{block_table, bt_stride_b, bt_blocks};
  EKV_REQUIRE(moments_workspace && mu_p && sigma_p && mu_g && sigma_g && mean_var && var_means &&
                  tau_hat && page_indices && counts && tau_floor && cache_seqlens && q && k &&
                  v && tau && out && workspace,
              "ekv_gaussian_paged_entmax_decode: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0,
              "ekv_gaussian_paged_entmax_decode: bad heads");
  EKV_REQUIRE(pages_for_stats > 0 && num_pages >= pages_for_stats && page_size > 0,
              "ekv_gaussian_paged_entmax_decode: bad page counts");
  EKV_REQUIRE(moments_workspace_bytes >=
                  ekv_gaussian_workspace_bytes(B, H, Hkv, D, pages_for_stats, dtype),
              "ekv_gaussian_paged_entmax_decode: moments workspace too small");
  EKV_REQUIRE(tau_hat_given || alpha == 2.0f || alpha == 1.5f || fabsf(alpha - 4.0f / 3.0f) < 1e-6f,
              "ekv_gaussian_paged_entmax_decode: tau-hat needs alpha in {2, 1.5, 4/3}");
  EKV_REQUIRE(tau_mode == 0 || tau_mode == 1, "ekv_gaussian_paged_entmax_decode: tau_mode %d",
              tau_mode);
  EKV_REQUIRE(iters >= 0 && max_tokens >= num_pages * page_size && kv_rows > 0,
              "ekv_gaussian_paged_entmax_decode: bad decode parameters");
  EKV_REQUIRE(workspace_bytes >= ekv_decode_workspace_bytes(B, H, Hkv, D, 1, max_tokens),
              "ekv_gaussian_paged_entmax_decode: workspace too small");
  if (int rc = check_kv_layout("ekv_gaussian_paged_entmax_decode", kv_stride_b, kv_stride_h,
                               kv_stride_row, blocks))
    return rc;
  hipStream_t s = (hipStream_t)stream;
  const int G = H / Hkv;
  const float* tau_start = tau_clamped ? tau_clamped : tau_hat;
  if (!one_workgroup_per_head(B * Hkv, seq_lens != nullptr)) {
    // few heads: moments, selection and a split decode as separate launches
    int rc = gauss::launch_finalize(moments_workspace, B, H, Hkv, pages_for_stats, mu_g, sigma_g,
                                    mean_var, var_means, tau_hat_given ? nullptr : tau_hat, alpha,
                                    n_tokens, tau_iters, tol, seq_lens, page_size, s);
    if (rc) return rc;
    rc = ekv_select_gaussian_pack(mu_p, sigma_p, tau_hat, sigma_g, B, H, Hkv, pages_for_stats,
                                  num_pages, alpha, auto_margins, safety_margin_z, z_page,
                                  z_page_low, z_page_high, threshold_excess_margin_fraction,
                                  page_indices, pi_stride_b, pi_stride_h, counts, tau_floor,
                                  cache_seqlens, page_size, last_page_size, tau_clamped, z_clamp,
                                  eps, effective_margins, seq_lens, stream);
    if (rc) return rc;
    return paged_decode(q, q_stride_b, q_stride_h, k, v, kv_stride_b, kv_stride_h, kv_stride_row,
                        kv_rows, page_indices, pi_stride_b, pi_stride_h, num_pages, cache_seqlens,
                        Hkv, 1, q_seqlens, alibi_slopes, tau_start, tau, tau_mode, iters, out,
                        out_stride_b, out_stride_h, alpha, qscale, page_size, B, H, Hkv, D,
                        splits_for(max_tokens), max_tokens, workspace, workspace_bytes, dtype,
                        stream, seq_lens != nullptr, nullptr, 0, 0, blocks);
  }
  DecodeArgs a = make_decode_args(q, q_stride_b, q_stride_h, k, v, kv_stride_b, kv_stride_h,
                                  kv_stride_row, kv_rows, page_indices, pi_stride_b, pi_stride_h,
                                  num_pages, cache_seqlens, Hkv, 1, q_seqlens, alibi_slopes,
                                  tau_start, tau, tau_mode, iters, out, out_stride_b,
                                  out_stride_h, alpha, qscale, page_size, H, Hkv, 1, max_tokens,
                                  workspace, blocks);
  a.scores_ready = 0;
  GaussArgs f;
  gauss::SelectArgs& sel = f.sel;
  sel.mu_p = mu_p;
  sel.sigma_p = sigma_p;
  sel.B = B;
  sel.H = H;
  sel.Hkv = Hkv;
  sel.pages = pages_for_stats;
  sel.num_pages = num_pages;
  sel.am1 = (float)(alpha - 1.0);
  sel.auto_margins = auto_margins;
  sel.smz = safety_margin_z;
  sel.z_page = z_page;
  sel.z_page_low = z_page_low;
  sel.z_page_high = z_page_high;
  sel.frac = threshold_excess_margin_fraction;
  sel.page_indices = page_indices;
  sel.pisb = pi_stride_b;
  sel.pish = pi_stride_h;
  sel.counts = counts;
  sel.tau_floor = tau_floor;
  sel.cache_seqlens = cache_seqlens;
  sel.page_size = page_size;
  sel.last_page_size = last_page_size;
  sel.tau_clamped = tau_clamped;
  sel.z_clamp = z_clamp;
  sel.eps = eps;
  sel.eff = effective_margins;
  sel.seq_lens = seq_lens;
  f.partials = (const float4*)moments_workspace;
  f.splits = gauss::moment_splits(B * Hkv, pages_for_stats, H / Hkv, seq_lens != nullptr);
  f.mu_g = mu_g;
  f.sigma_g = sigma_g;
  f.mean_var = mean_var;
  f.var_means = var_means;
  f.tau_hat = tau_hat;
  f.tau_hat_given = tau_hat_given;
  f.tau_alpha = fabsf(alpha - 4.0f / 3.0f) < 1e-6f ? 4.0f / 3.0f : alpha;
  f.n_tokens = (float)n_tokens;
  f.log_n_factor = (float)sqrt(2.0 * log((double)n_tokens + 1.0));
  f.tau_iters = tau_iters;
  f.tol = tol;
  if (G >= 4 && 2 * B * Hkv <= device_cus()) {
    // two workgroups per (b, kv head) share large selections' K scoring; the
    // arrival words follow the workspace's scores (a fresh tag per call, as
    // in the paired top-k launch)
    static std::atomic<unsigned long long> launches{0};
    f.pair_cnt = (unsigned long long*)((char*)workspace +
                                       ((int64_t)B * H * max_tokens * 4 + 255) / 256 * 256);
    f.pair_tag = ((launches.fetch_add(1, std::memory_order_relaxed) + 1) *
                  0xD1B54A32D192ED03ull) | 1ull;
  }
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    return dispatch_group(G, [&](auto gv) {
      return dec::Launch<T, decltype(gv)::value>::gaussian(a, f, B, Hkv, D, max_tokens, s);
    });
  });
}

// ---------------------------------------------------------------------------
// dense (non-paged) decode: kernels/adadecode.py:754-1016
// ---------------------------------------------------------------------------

namespace {

// The contiguous cache is read through the paged decode with an identity page
// table; pages are grouped so that the table always fits the LDS staging
// table (kTablePages entries).
struct DenseGeom {
  int page_size, n_slots, max_tokens;
  int64_t score_bytes, total_bytes;
};

DenseGeom dense_geom(int B, int H, int64_t kv_rows) {
  DenseGeom g;
  g.page_size = 16;
  while ((kv_rows + g.page_size - 1) / g.page_size > kTablePages) g.page_size *= 2;
  g.n_slots = (int)((kv_rows + g.page_size - 1) / g.page_size);
  g.max_tokens = g.n_slots * g.page_size;
  g.score_bytes = ekv_decode_workspace_bytes(B, H, H, 0, 1, g.max_tokens);
  g.total_bytes = g.score_bytes + ((int64_t)g.n_slots * 4 + 255) / 256 * 256;
  return g;
}

// Heads longer than this are scored by many workgroups each (the split
// path): one workgroup per head would stream all of its keys from one CU.
constexpr int kDenseHeadTokens = 8192;

__global__ void iota_kernel(int32_t* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = i;
}

}  // namespace

extern "C" int64_t ekv_dense_decode_workspace_bytes(int B, int H, int64_t kv_rows) {
  if (B <= 0 || H <= 0 || kv_rows <= 0 || kv_rows > INT_MAX / 2) return -1;
  return dense_geom(B, H, kv_rows).total_bytes;
}

extern "C" int ekv_dense_entmax_decode(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k, const void* v,
    int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_row, int64_t kv_rows,
    const int32_t* cache_seqlens, const int32_t* token_positions, int64_t pos_stride_b,
    int64_t pos_stride_h, const int32_t* q_seqlens, const float* alibi_slopes, float* tau,
    int iters, void* out, int64_t out_stride_b, int64_t out_stride_h, float alpha, float qscale,
    int B, int H, int Hkv, int D, void* workspace, int64_t workspace_bytes, int dtype,
    void* stream) {
  EKV_REQUIRE(q && k && v && cache_seqlens && tau && out && workspace,
              "ekv_dense_entmax_decode: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "ekv_dense_entmax_decode: bad heads");
  EKV_REQUIRE(kv_rows > 0 && kv_rows <= INT_MAX / 2, "ekv_dense_entmax_decode: bad kv_rows");
  const DenseGeom g = dense_geom(B, H, kv_rows);
  EKV_REQUIRE(workspace_bytes >= g.total_bytes, "ekv_dense_entmax_decode: workspace too small");
  int32_t* table = (int32_t*)((char*)workspace + g.score_bytes);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(iota_kernel, dim3((g.n_slots + 255) / 256), dim3(256), 0, s, table,
                     g.n_slots);
  if (int rc = check_launch("iota_kernel")) return rc;
  return paged_decode(q, q_stride_b, q_stride_h, k, v, kv_stride_b, kv_stride_h, kv_stride_row,
                      kv_rows, table, 0, 0, g.n_slots, cache_seqlens, 1, 0, q_seqlens,
                      alibi_slopes, nullptr, tau, 0, iters, out, out_stride_b, out_stride_h,
                      alpha, qscale, g.page_size, B, H, Hkv, D, splits_for(g.max_tokens),
                      g.max_tokens, workspace, g.score_bytes, dtype, stream,
                      g.max_tokens > kDenseHeadTokens,
                      alibi_slopes ? token_positions : nullptr, pos_stride_b, pos_stride_h);
}
