// Gaussian-aware page selection: page score moments, the tau-hat solvers,
// threshold selection + pack, tau clamp and compacted lengths.
//
//   moments_kernel          kernels/gaussian_page_stats.py:8-121 and
//                           gaussian_utils.py:130-161: per page
//                           mu_p = sum_d (q_d/sqrt(D)) kmean_pd,
//                           var_p = sum_d (q_d/sqrt(D))^2 kstd_pd^2, and each
//                           workgroup's partial sums of the global moments.
//   finalize_kernel         gaussian_utils.py:155-181: global moments per
//                           head from the partials, single-Gaussian tau-hat.
//   tau_single_gaussian     kernels/tau_solver_gpu.py:20-125.
//   tau_page_mixture        kernels/tau_mixture_solver_triton.py:9-165.
//   select_pack_kernel      kernels/selection_pack.py:113-198 (threshold,
//                           ascending pack, last-page sentinel),
//                           gaussian_utils.py:163-169 (auto margins on
//                           device, no host sync), kernels/tau_clamp.py:8-73
//                           and kernels/selection_pack.py:7-20, fused.
//
// Under GQA (H = G * Hkv) every query head keeps its own moments, tau-hat and
// tau floor; the page table of a kv head is the union of its query heads'
// selections (for G = 1 this is the reference's per-head selection).
#include <atomic>

#include "ekv_common.h"
#include "gaussian_device.h"
#include "../../include/entmaxkv.h"

using namespace ekv;
using namespace ekv::gauss;

namespace {

constexpr int kThreads = 256;
// pages per row segment per round (two rounds in flight): one measured
// slightly faster than two and four at the headline shape
constexpr int kMomentUnroll = 1;

template <typename T, int LPR, int G, bool kNt>
__global__ __launch_bounds__(moment_threads(G)) void moments_kernel(MomentsArgs a) {
  const int bkv = blockIdx.y;
  if (a.pages_per_split * G <= kMomentLdsEntries)
    moments_partial_block<T, LPR, G, moment_threads(G), kMomentUnroll, true, kNt>(
        a, bkv / a.Hkv, bkv % a.Hkv, blockIdx.x);
  else
    moments_partial_block<T, LPR, G, moment_threads(G), kMomentUnroll, false, kNt>(
        a, bkv / a.Hkv, bkv % a.Hkv, blockIdx.x);
}

// One wave per (b, h): global moments from the partials (reduced by the
// first split_lanes(splits) lanes) and (optional) the single-Gaussian tau-hat.
__global__ __launch_bounds__(kThreads) void finalize_kernel(const float4* partials, int splits,
                                                            int pages, int count, float* mu_g,
                                                            float* sigma_g, float* mean_var,
                                                            float* var_means, float* tau_hat,
                                                            float alpha, float n_tokens,
                                                            float log_n_factor, int iters,
                                                            float tol, const int32_t* seq_lens,
                                                            int page_size, int H) {
  const int head = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (head >= count) return;
  const TauGeom tg = tau_geom(seq_lens, head / H, page_size, pages, n_tokens, log_n_factor);
  const int lane = threadIdx.x & 63;
  const int s2 = split_lanes(splits);
  float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
  if (lane < splits) x = partials[(int64_t)head * splits + lane];
  if (lane >= s2) x = make_float4(0.f, 0.f, 0.f, 0.f);
  x = reduce_splits(x, s2);
  x.x = __shfl(x.x, 0);
  x.y = __shfl(x.y, 0);
  x.z = __shfl(x.z, 0);
  const Moments m = finalize_moments(x, tg.pages);
  float th = 0.f;
  if (tau_hat) th = solve_single_gaussian_wave(m.mu_g, m.sigma_g, tg.n, alpha, tg.lnf, iters, tol);
  if (lane == 0) {
    mu_g[head] = m.mu_g;
    sigma_g[head] = m.sigma_g;
    mean_var[head] = m.mean_var;
    var_means[head] = m.var_means;
    if (tau_hat) tau_hat[head] = th;
  }
}

__global__ void tau_single_kernel(const float* mu, const float* sigma, float* out, int count, float n,
                                  float alpha, float lnf, int iters, float tol) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  out[i] = solve_single_gaussian(mu[i], sigma[i], n, alpha, lnf, iters, tol);
}

// ---------------------------------------------------------------------------
// page-mixture tau-hat (ALiBi), one workgroup per row
// ---------------------------------------------------------------------------

__device__ void mixture_eval(const float* __restrict__ mu, const float* __restrict__ sg, int pages,
                             float cnt, float alpha, float tau, float* scratch, float& f, float& f1,
                             float& f2) {
  float e = 0.f, d1 = 0.f, d2 = 0.f;
  for (int p = threadIdx.x; p < pages; p += blockDim.x) {
    float x, y, z;
    gaussian_terms(tau, mu[p], fmaxf(sg[p], 1.0e-6f), cnt, alpha, x, y, z);
    e += x;
    d1 += y;
    d2 += z;
  }
  f = block_sum(e, scratch) - 1.0f;
  f1 = block_sum(d1, scratch);
  f2 = block_sum(d2, scratch);
}

__global__ __launch_bounds__(kThreads) void tau_mixture_kernel(const float* mu_p, const float* sigma_p,
                                                               float* out, int stride, float cnt,
                                                               float alpha, int iters, float tol,
                                                               const int32_t* seq_lens,
                                                               int rows_per_seq, int page_size) {
  __shared__ float scratch[16];
  const int row = blockIdx.x;
  const float* mu = mu_p + (int64_t)row * stride;
  const float* sg = sigma_p + (int64_t)row * stride;
  // a ragged batch mixes only this sequence's statistics pages
  const int pages =
      seq_lens ? min(seq_pages(seq_lens[row / rows_per_seq], page_size).stat_pages, stride) : stride;
  const float a = alpha - 1.0f;
  float my = -INFINITY, ms = 0.f;
  for (int p = threadIdx.x; p < pages; p += blockDim.x) {
    my = fmaxf(my, a * mu[p]);
    ms = fmaxf(ms, a * fmaxf(sg[p], 1.0e-6f));
  }
  __shared__ float smax[2][kThreads / 64];
  my = wave_max(my);
  ms = wave_max(ms);
  if ((threadIdx.x & 63) == 0) {
    smax[0][threadIdx.x >> 6] = my;
    smax[1][threadIdx.x >> 6] = ms;
  }
  __syncthreads();
  my = -INFINITY;
  ms = 0.f;
  for (int w = 0; w < kThreads / 64; ++w) {
    my = fmaxf(my, smax[0][w]);
    ms = fmaxf(ms, smax[1][w]);
  }
  ms = fmaxf(ms, 1.0e-6f);
  const float total = fmaxf(cnt * (float)pages, 1.0f);
  const float lnf = sqrtf(2.0f * logf(total + 1.0f));
  float radius = ms * (lnf + 8.0f);
  float lo = my - radius, hi = my + radius;
  float f, f1, f2;
  for (int i = 0; i < 8; ++i) {
    float fl, fh;
    mixture_eval(mu, sg, pages, cnt, alpha, lo, scratch, fl, f1, f2);
    mixture_eval(mu, sg, pages, cnt, alpha, hi, scratch, fh, f1, f2);
    if (fl <= 0.0f) lo -= radius;
    if (fh > 0.0f) hi += radius;
    radius *= 2.0f;
  }
  float t = 0.5f * (lo + hi);
  for (int it = 0; it < iters; ++it) {
    mixture_eval(mu, sg, pages, cnt, alpha, t, scratch, f, f1, f2);
    const float mid = 0.5f * (lo + hi);
    const float den = 2.0f * f1 * f1 - f * f2;
    const float step = fabsf(den) > 1.0e-18f ? 2.0f * f * f1 / den : f / fminf(f1, -1.0e-12f);
    float cand = t - step;
    if (!(cand == cand && fabsf(cand) < 1.0e20f && cand > lo && cand < hi)) cand = mid;
    float fc, u1, u2;
    mixture_eval(mu, sg, pages, cnt, alpha, cand, scratch, fc, u1, u2);
    if (fc > 0.0f) lo = cand;
    else hi = cand;
    if (fabsf(fc) <= tol) {
      const bool small = fabsf(cand - t) <= 1.0e-6f * fmaxf(1.0f, fabsf(t));
      t = cand;
      if (small) break;
    } else {
      t = 0.5f * (lo + hi);
    }
  }
  if (threadIdx.x == 0) out[row] = (pages > 0 && cnt > 0.f) ? t : 0.0f;
}

// ---------------------------------------------------------------------------
// threshold selection + pack + clamp + compacted lengths
// ---------------------------------------------------------------------------

// Standalone selection launch: one workgroup per (b, kv head); the mean
// sigma_g of the automatic margins is summed from the sigma_g array.
template <int G>
__global__ __launch_bounds__(kThreads) void select_pack_kernel(SelectArgs a, const float* tau_hat,
                                                              const float* sigma_g) {
  __shared__ float scratch[16];
  const int bkv = blockIdx.x;
  const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
  float sbar = 0.f;
  if (a.auto_margins) {
    float s = 0.f;
    const int nh = a.B * a.H;
    for (int i = threadIdx.x; i < nh; i += kThreads) s += sigma_g[i];
    sbar = block_sum(s, scratch) / (float)nh;
  }
  float th[G], sg[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    th[g] = tau_hat[b * a.H + kvh * G + g];
    sg[g] = sigma_g[b * a.H + kvh * G + g];
  }
  select_pack_block<G, kThreads>(a, b, kvh, sbar, th, sg, nullptr, 0, nullptr);
}

// Standalone clamp over a caller-provided page list (kernels/tau_clamp.py:8-73).
__global__ __launch_bounds__(kThreads) void tau_clamp_kernel(
    const float* tau, const float* mu_p, const float* sigma_p, const int32_t* page_indices,
    int64_t pisb, int64_t pish, int n_slots, const int32_t* num_selected, int64_t nsb, int64_t nsh,
    const float* tau_floor, float* out, int H, int Hsel, int pages, float am1, float z_clamp,
    float eps) {
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh % H;
  const int hs = h / (H / Hsel);
  const int32_t* pi = page_indices + b * pisb + hs * pish;
  const int nsel = num_selected[b * nsb + hs * nsh];
  const float* mu = mu_p + (int64_t)bh * pages;
  const float* sg = sigma_p + (int64_t)bh * pages;
  float m = -INFINITY;
  for (int i = threadIdx.x; i < n_slots; i += blockDim.x) {
    const int p = pi[i];
    if (i < nsel && p >= 0 && p < pages)
      m = fmaxf(m, fma_rn(mul_rn(z_clamp, sg[p]), 0.3333333333333333f, mu[p]));
  }
  __shared__ float cm[kThreads / 64];
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) cm[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float mx = -INFINITY;
    for (int w = 0; w < kThreads / 64; ++w) mx = fmaxf(mx, cm[w]);
    float up = fma_rn(am1, mx, -eps);
    if (tau_floor) up = fmaxf(up, tau_floor[bh]);
    out[bh] = (mx > -3.0e38f) ? fminf(tau[bh], up) : tau[bh];
  }
}

__global__ void seqlens_kernel(const int32_t* counts, int32_t* out, int n, int ps, int last) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = max(counts[i] - 1, 0) * ps + last;
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

}  // namespace

int ekv::gauss::launch_finalize(const void* partials, int B, int H, int Hkv, int pages,
                                float* mu_g, float* sigma_g, float* mean_var, float* var_means,
                                float* tau_hat, float alpha, int n_tokens, int tau_iters, float tol,
                                const int32_t* seq_lens, int page_size, hipStream_t stream) {
  const int count = B * H;
  const float al = fabsf(alpha - 4.0f / 3.0f) < 1e-6f ? 4.0f / 3.0f : alpha;
  const float lnf = (float)sqrt(2.0 * log((double)n_tokens + 1.0));
  hipLaunchKernelGGL(finalize_kernel, dim3((count + kThreads / 64 - 1) / (kThreads / 64)),
                     dim3(kThreads), 0, stream, (const float4*)partials,
                     moment_splits(B * Hkv, pages, H / Hkv, seq_lens != nullptr), pages, count, mu_g, sigma_g, mean_var,
                     var_means, tau_hat, al, (float)n_tokens, lnf, tau_iters, tol, seq_lens,
                     page_size, H);
  return check_launch("finalize_kernel");
}

extern "C" int64_t ekv_gaussian_workspace_bytes(int B, int H, int Hkv, int D, int pages, int dtype) {
  (void)D;
  (void)dtype;
  if (B <= 0 || H <= 0 || Hkv <= 0 || pages <= 0) return 0;
  // sized for the ragged split count, which is never below the uniform one
  const int splits = moment_splits(B * Hkv, pages, H / Hkv, true);
  return ((int64_t)B * H * splits * 16 + 255) / 256 * 256;
}

extern "C" int ekv_gaussian_moments(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kmean, const void* kstd,
    int64_t s_stride_b, int64_t s_stride_h, int64_t s_stride_page, int pages_for_stats,
    const float* alibi_slopes, int page_size, int seq_len, int n_tokens, const int32_t* seq_lens,
    float* mu_p, float* sigma_p, int B, int H, int Hkv, int D, void* workspace,
    int64_t workspace_bytes, int dtype, void* stream) {
  EKV_REQUIRE(q && kmean && kstd && mu_p && sigma_p && workspace,
              "ekv_gaussian_moments: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "ekv_gaussian_moments: bad heads");
  EKV_REQUIRE(pages_for_stats > 0, "ekv_gaussian_moments: pages_for_stats must be positive");
  EKV_REQUIRE(workspace_bytes >= ekv_gaussian_workspace_bytes(B, H, Hkv, D, pages_for_stats, dtype),
              "ekv_gaussian_moments: workspace too small");
  MomentsArgs a;
  a.q = q;
  a.qsb = q_stride_b;
  a.qsh = q_stride_h;
  a.kmean = kmean;
  a.kstd = kstd;
  a.ssb = s_stride_b;
  a.ssh = s_stride_h;
  a.ssp = s_stride_page;
  a.pages = pages_for_stats;
  a.splits = moment_splits(B * Hkv, pages_for_stats, H / Hkv, seq_lens != nullptr);
  a.pages_per_split = (pages_for_stats + a.splits - 1) / a.splits;
  a.H = H;
  a.Hkv = Hkv;
  a.scale = (float)(1.0 / sqrt((double)D));
  a.slopes = alibi_slopes;
  a.page_size = page_size;
  a.q_pos = seq_len - 1;
  a.stats_len = n_tokens;
  a.mu_p = mu_p;
  a.sigma_p = sigma_p;
  a.partials = (float4*)workspace;
  a.seq_lens = seq_lens;
  {
    // consecutive launches scan in opposite orders (the reason is the
    // criticality scan's, next_scan_order)
    static std::atomic<unsigned> scans{0};
    a.rev = (int)(scans.fetch_add(1, std::memory_order_relaxed) & 1u);
  }
  a.nt = stream_nt(B, Hkv, pages_for_stats, D, dtype) ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    return dispatch_lpr<T>(D, [&](auto lpr) {
      constexpr int LPR = decltype(lpr)::value;
      return dispatch_group(H / Hkv, [&](auto gv) {
        constexpr int G = decltype(gv)::value;
        if (a.nt)
          hipLaunchKernelGGL((moments_kernel<T, LPR, G, true>), dim3(a.splits, B * Hkv),
                             dim3(moment_threads(G)), 0, s, a);
        else
          hipLaunchKernelGGL((moments_kernel<T, LPR, G, false>), dim3(a.splits, B * Hkv),
                             dim3(moment_threads(G)), 0, s, a);
        return check_launch("moments_kernel");
      });
    });
  });
}

extern "C" int ekv_gaussian_page_stats(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kmean, const void* kstd,
    int64_t s_stride_b, int64_t s_stride_h, int64_t s_stride_page, int pages_for_stats,
    const float* alibi_slopes, int page_size, int seq_len, float* mu_p, float* sigma_p, float* mu_g,
    float* sigma_g, float* mean_var, float* var_means, float* tau_hat, float alpha, int n_tokens,
    int tau_iters, float tol, const int32_t* seq_lens, int B, int H, int Hkv, int D,
    void* workspace, int64_t workspace_bytes, int dtype, void* stream) {
  EKV_REQUIRE(mu_g && sigma_g && mean_var && var_means, "ekv_gaussian_page_stats: null pointer");
  EKV_REQUIRE(!tau_hat || alpha == 2.0f || alpha == 1.5f || fabsf(alpha - 4.0f / 3.0f) < 1e-6f,
              "ekv_gaussian_page_stats: tau-hat needs alpha in {2, 1.5, 4/3}");
  int rc = ekv_gaussian_moments(q, q_stride_b, q_stride_h, kmean, kstd, s_stride_b, s_stride_h,
                                s_stride_page, pages_for_stats, alibi_slopes, page_size, seq_len,
                                n_tokens, seq_lens, mu_p, sigma_p, B, H, Hkv, D, workspace,
                                workspace_bytes, dtype, stream);
  if (rc) return rc;
  return launch_finalize(workspace, B, H, Hkv, pages_for_stats, mu_g, sigma_g, mean_var,
                         var_means, tau_hat, alpha, n_tokens, tau_iters, tol, seq_lens, page_size,
                         (hipStream_t)stream);
}

extern "C" int ekv_tau_single_gaussian(const float* mu_g, const float* sigma_g, float* tau_out,
                                       int count, int n_tokens, float alpha, int iterations,
                                       float tol, void* stream) {
  EKV_REQUIRE(mu_g && sigma_g && tau_out && count >= 0 && n_tokens >= 0,
              "ekv_tau_single_gaussian: bad arguments");
  if (count == 0) return EKV_OK;
  const float lnf = (float)sqrt(2.0 * log((double)n_tokens + 1.0));
  hipLaunchKernelGGL(tau_single_kernel, dim3((count + 255) / 256), dim3(256), 0,
                     (hipStream_t)stream, mu_g, sigma_g, tau_out, count, (float)n_tokens, alpha,
                     lnf, iterations, tol);
  return check_launch("tau_single_kernel");
}

extern "C" int ekv_tau_page_mixture(const float* mu_p, const float* sigma_p, float* tau_out,
                                    int rows, int pages, float page_count, float alpha, int max_iter,
                                    float tol, const int32_t* seq_lens, int rows_per_seq,
                                    int page_size, void* stream) {
  EKV_REQUIRE(mu_p && sigma_p && tau_out && rows >= 0 && pages > 0 && page_count > 0.f,
              "ekv_tau_page_mixture: bad arguments");
  EKV_REQUIRE(!seq_lens || (rows_per_seq > 0 && page_size > 0),
              "ekv_tau_page_mixture: ragged rows need rows_per_seq and page_size");
  if (rows == 0) return EKV_OK;
  hipLaunchKernelGGL(tau_mixture_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, mu_p,
                     sigma_p, tau_out, pages, page_count, alpha, max_iter, tol, seq_lens,
                     rows_per_seq, page_size);
  return check_launch("tau_mixture_kernel");
}

extern "C" int ekv_select_gaussian_pack(
    const float* mu_p, const float* sigma_p, const float* tau_hat, const float* sigma_g, int B,
    int H, int Hkv, int pages_for_stats, int num_pages, float alpha, int auto_margins,
    float safety_margin_z, float z_page, float z_page_low, float z_page_high,
    float threshold_excess_margin_fraction, int32_t* page_indices, int64_t pi_stride_b,
    int64_t pi_stride_h, int32_t* counts, float* tau_floor, int32_t* cache_seqlens, int page_size,
    int last_page_size, float* tau_clamped, float z_clamp, float eps, float* effective_margins,
    const int32_t* seq_lens, void* stream) {
  EKV_REQUIRE(mu_p && sigma_p && tau_hat && sigma_g && page_indices && counts && tau_floor,
              "ekv_select_gaussian_pack: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "ekv_select_gaussian_pack: bad heads");
  EKV_REQUIRE(pages_for_stats > 0 && num_pages >= pages_for_stats,
              "ekv_select_gaussian_pack: pages_for_stats and num_pages must be positive");
  SelectArgs a;
  a.mu_p = mu_p;
  a.sigma_p = sigma_p;
  a.B = B;
  a.H = H;
  a.Hkv = Hkv;
  a.pages = pages_for_stats;
  a.num_pages = num_pages;
  a.am1 = (float)(alpha - 1.0);
  a.auto_margins = auto_margins;
  a.smz = safety_margin_z;
  a.z_page = z_page;
  a.z_page_low = z_page_low;
  a.z_page_high = z_page_high;
  a.frac = threshold_excess_margin_fraction;
  a.page_indices = page_indices;
  a.pisb = pi_stride_b;
  a.pish = pi_stride_h;
  a.counts = counts;
  a.tau_floor = tau_floor;
  a.cache_seqlens = cache_seqlens;
  a.page_size = page_size;
  a.last_page_size = last_page_size;
  a.tau_clamped = tau_clamped;
  a.z_clamp = z_clamp;
  a.eps = eps;
  a.eff = effective_margins;
  a.seq_lens = seq_lens;
  hipStream_t s = (hipStream_t)stream;
  return dispatch_group(H / Hkv, [&](auto gv) {
    constexpr int G = decltype(gv)::value;
    hipLaunchKernelGGL((select_pack_kernel<G>), dim3(B * Hkv), dim3(kThreads), 0, s, a, tau_hat,
                       sigma_g);
    return check_launch("select_pack_kernel");
  });
}

extern "C" int ekv_tau_clamp(const float* tau, const float* mu_p, const float* sigma_p,
                             const int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h,
                             int n_slots, const int32_t* num_selected, int64_t ns_stride_b,
                             int64_t ns_stride_h, const float* tau_floor, float* out, int B, int H,
                             int Hsel, int pages_for_stats, float alpha, float z_clamp, float eps,
                             void* stream) {
  EKV_REQUIRE(tau && mu_p && sigma_p && page_indices && num_selected && out,
              "ekv_tau_clamp: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hsel > 0 && H % Hsel == 0 && n_slots >= 0 && pages_for_stats > 0,
              "ekv_tau_clamp: bad sizes");
  hipLaunchKernelGGL(tau_clamp_kernel, dim3(B * H), dim3(kThreads), 0, (hipStream_t)stream, tau,
                     mu_p, sigma_p, page_indices, pi_stride_b, pi_stride_h, n_slots, num_selected,
                     ns_stride_b, ns_stride_h, tau_floor, out, H, Hsel, pages_for_stats,
                     (float)(alpha - 1.0), z_clamp, eps);
  return check_launch("tau_clamp_kernel");
}

extern "C" int ekv_cache_seqlens_from_counts(const int32_t* counts, int32_t* cache_seqlens, int n,
                                             int page_size, int last_page_size, void* stream) {
  EKV_REQUIRE(counts && cache_seqlens && n >= 0, "ekv_cache_seqlens_from_counts: bad arguments");
  if (n == 0) return EKV_OK;
  hipLaunchKernelGGL(seqlens_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     counts, cache_seqlens, n, page_size, last_page_size);
  return check_launch("seqlens_kernel");
}
