// Device-side building blocks of the Gaussian-aware page selection, shared by
// the standalone launches (gaussian_select.hip) and the fused select + decode
// launch (paged_decode.hip).
//
//   gaussian_terms / solve_*      tau_solver.py:31-120, 347-412 and
//                                 kernels/tau_solver_gpu.py:20-125
//   moments_partial_block         kernels/gaussian_page_stats.py:8-121 and
//                                 gaussian_utils.py:130-161 (per-page moments
//                                 and this workgroup's share of the global sums)
//   finalize_moments              gaussian_utils.py:155-161
//   select_pack_block             kernels/selection_pack.py:113-198,
//                                 gaussian_utils.py:163-169 (automatic
//                                 margins), kernels/tau_clamp.py:8-73,
//                                 kernels/selection_pack.py:7-20
//
// The global moments of a head are reduced from per-workgroup partial sums
// (Sum mu_p, Sum mu_p^2, Sum sigma_p^2) that the moments launch writes with
// plain stores; whoever needs mu_g / sigma_g sums a head's partials in a fixed
// order, so every consumer derives bit-identical values and no workgroup ever
// waits for another.
#pragma once

#include "ekv_common.h"

namespace ekv {
namespace gauss {

// Threads per workgroup of the moments launch for GQA group G: 1024 (one
// workgroup streaming a head's contiguous statistics measured faster than
// four of 256 threads) unless the G query heads' registers need more than
// 1024 threads leave (G >= 4: 256 threads).
constexpr int moment_threads(int G) { return G <= 2 ? 1024 : 256; }

// Workgroups per (b, kv head) of the moments launch: about 256K threads in
// all, at least 256 pages each, at most 64 per head.  A ragged batch
// (`ragged`: per-sequence lengths) takes 256 pages per workgroup of the
// longest row whatever the thread count, so the long sequences do not leave
// a few workgroups streaming long after the rest (a shorter sequence's extra
// workgroups have no pages and exit).  Every launch that reads the partials
// of one moments launch must pass the same `ragged`.
inline int moment_splits(int bkv, int pages, int G, bool ragged = false) {
  const int target = (256 * 1024) / moment_threads(G);
  int s = (target + bkv - 1) / bkv;
  const int by_pages = (pages + 255) / 256;
  if (s > by_pages || ragged) s = by_pages;
  if (s > 64) s = 64;
  return s < 1 ? 1 : s;
}

// Host launcher (gaussian_select.hip) of the global moments and tau-hat from
// the moments launch's partials (tau_hat may be null); the fused entry point's
// fallback uses it.
int launch_finalize(const void* partials, int B, int H, int Hkv, int pages, float* mu_g,
                    float* sigma_g, float* mean_var, float* var_means, float* tau_hat, float alpha,
                    int n_tokens, int tau_iters, float tol, const int32_t* seq_lens,
                    int page_size, hipStream_t stream);

__device__ __forceinline__ float normal_pdf(float x) {
  return expf(-0.5f * x * x) * 0.3989422804014327f;
}
// Phi(x) = 0.5 * erfc(-x / sqrt(2)): equal to 0.5 * (1 + erf(x / sqrt(2))) but
// without the cancellation of 1 + erf in the lower tail.
__device__ __forceinline__ float normal_cdf(float x) {
  return 0.5f * erfcf(-x * 0.7071067811865476f);
}

// f(tau) = n*E[[(alpha-1)S - tau]_+^(1/(alpha-1))] for S ~ N(mu, sigma^2)
// (count weight `n`), with first and second derivatives in tau.  The third
// moment used for alpha = 4/3 is the reference's expression
// (tau_solver.py:104-107).
__device__ __forceinline__ void gaussian_terms(float tau, float mu, float sigma, float n,
                                               float alpha, float& e, float& d1, float& d2) {
  const float a = alpha - 1.0f;
  const float sy = fmaxf(a * sigma, 1.0e-10f);
  const float my = a * mu - tau;
  const float t = my / sy;
  const float ph = normal_pdf(t);
  const float Ph = normal_cdf(t);
  const float m0 = Ph;
  const float m1 = my * Ph + sy * ph;
  const float m2 = (my * my + sy * sy) * Ph + my * sy * ph;
  if (alpha == 2.0f) {
    e = n * m1;
    d1 = -n * m0;
    d2 = n * ph / sy;
  } else if (alpha == 1.5f) {
    e = n * m2;
    d1 = -2.0f * n * m1;
    d2 = 2.0f * n * m0;
  } else {
    const float m3 = (my * my * my + 3.0f * my * sy * sy) * Ph + (sy * sy * sy + 2.0f * my * my * sy) * ph;
    e = n * m3;
    d1 = -3.0f * n * m2;
    d2 = 6.0f * n * m1;
  }
}

// One bracketed Halley step with bisection fallback (tau_solver.py:380-410):
// updates (t, lo, hi); returns true once a candidate is accepted after a step
// below 1e-6 * max(1, |t|).
__device__ __forceinline__ bool halley_bracket_step(float& t, float& lo, float& hi, float mu,
                                                    float sigma, float n, float alpha, float tol) {
  float e, f1, f2;
  gaussian_terms(t, mu, sigma, n, alpha, e, f1, f2);
  const float f = e - 1.0f;
  const float mid = 0.5f * (lo + hi);
  const float den = 2.0f * f1 * f1 - f * f2;
  const float step = fabsf(den) > 1.0e-18f ? 2.0f * f * f1 / den : f / fminf(f1, -1.0e-12f);
  float cand = t - step;
  if (!(cand == cand && fabsf(cand) < 1.0e20f && cand > lo && cand < hi)) cand = mid;
  float ec, u1, u2;
  gaussian_terms(cand, mu, sigma, n, alpha, ec, u1, u2);
  const float fc = ec - 1.0f;
  if (fc > 0.0f) lo = cand;
  else hi = cand;
  if (fabsf(fc) <= tol) {
    const bool small = fabsf(cand - t) <= 1.0e-6f * fmaxf(1.0f, fabsf(t));
    t = cand;
    return small;
  }
  t = 0.5f * (lo + hi);
  return false;
}

// Single-Gaussian tau-hat solved by one lane: the reference's bracket
// (alpha-1)mu +- (alpha-1)sigma(sqrt(2 ln(n+1)) + 8) and up to `iterations`
// bracketed Halley steps, stopping early once a step is accepted.
__device__ __forceinline__ float solve_single_gaussian(float mu, float sigma, float n, float alpha,
                                                       float log_n_factor, int iterations,
                                                       float tol) {
  sigma = fmaxf(sigma, 1.0e-6f);
  const float a = alpha - 1.0f;
  const float radius = a * sigma * (log_n_factor + 8.0f);
  float lo = a * mu - radius, hi = a * mu + radius;
  float t = 0.5f * (lo + hi);
  for (int it = 0; it < iterations; ++it)
    if (halley_bracket_step(t, lo, hi, mu, sigma, n, alpha, tol)) break;
  return t;
}

// The same root solved by a whole wave (every lane returns it): two rounds of
// a 64-point bracket search (f is decreasing in tau, so the positive lanes
// form a prefix; the bracket shrinks 65x per round), then Halley steps with
// bisection fallback from the middle of the final bracket, one evaluation of
// f per step, until |f(t)| <= tol and the next step is below
// 1e-6 * max(1, |t|) (at most `iterations`, capped at 8).  About five
// function evaluations in all.
__device__ __forceinline__ float solve_single_gaussian_wave(float mu, float sigma, float n,
                                                            float alpha, float log_n_factor,
                                                            int iterations, float tol) {
  sigma = fmaxf(sigma, 1.0e-6f);
  const float a = alpha - 1.0f;
  const float radius = a * sigma * (log_n_factor + 8.0f);
  float lo = a * mu - radius, hi = a * mu + radius;
  const int lane = threadIdx.x & 63;
#pragma unroll 1
  for (int r = 0; r < 2; ++r) {
    const float w = (hi - lo) * (1.0f / 65.0f);
    const float x = fmaf(w, (float)(lane + 1), lo);
    float e, d1, d2;
    gaussian_terms(x, mu, sigma, n, alpha, e, d1, d2);
    const uint64_t pos = __ballot(e - 1.0f > 0.0f);
    // last lane with f > 0 (lanes past it read f <= 0)
    const int k = pos ? 64 - __builtin_clzll(pos) : 0;
    const float nlo = k > 0 ? fmaf(w, (float)k, lo) : lo;
    const float nhi = k < 64 ? fmaf(w, (float)(k + 1), lo) : hi;
    lo = nlo;
    hi = fmaxf(nhi, nlo);
  }
  float t = 0.5f * (lo + hi);
  const int steps = iterations < 8 ? iterations : 8;
  for (int it = 0; it < steps; ++it) {
    float e, f1, f2;
    gaussian_terms(t, mu, sigma, n, alpha, e, f1, f2);
    const float f = e - 1.0f;
    if (f > 0.0f) lo = t;
    else hi = t;
    const float den = 2.0f * f1 * f1 - f * f2;
    const float step = fabsf(den) > 1.0e-18f ? 2.0f * f * f1 / den : f / fminf(f1, -1.0e-12f);
    // converged at t: the test comes before the bracket check, since a step
    // this small can round onto the bracket edge
    // or stalled: a step or a bracket of a few ulps is fp32 noise in f
    // (the reference's moment formulas cancel), not progress
    const float scale_t = fmaxf(1.0f, fabsf(t));
    if ((fabsf(f) <= tol && fabsf(step) <= 1.0e-6f * scale_t) || fabsf(step) <= 2.4e-7f * scale_t ||
        hi - lo <= 4.8e-7f * scale_t)
      break;
    float cand = t - step;
    if (!(cand == cand && fabsf(cand) < 1.0e20f && cand > lo && cand < hi)) cand = 0.5f * (lo + hi);
    t = cand;
  }
  return t;
}

// ---------------------------------------------------------------------------
// per-page moments and per-workgroup partial sums
// ---------------------------------------------------------------------------

struct MomentsArgs {
  const void* q;
  int64_t qsb, qsh;
  const void* kmean;
  const void* kstd;
  int64_t ssb, ssh, ssp;
  int pages;            // pages_for_stats
  int pages_per_split;  // pages handled by one workgroup
  int splits;           // workgroups per (b, kv head)
  int H, Hkv;
  float scale;          // 1/sqrt(D) in fp32
  const float* slopes;  // ALiBi [H] or null
  int page_size;
  int q_pos;            // seq_len - 1
  int stats_len;        // seq_len_for_stats
  float* mu_p;          // [B, H, pages]
  float* sigma_p;       // [B, H, pages]
  float4* partials;     // [B, H, splits] (Sum mu, Sum mu^2, Sum var, 0)
  const int32_t* seq_lens;  // [B] per-sequence lengths (ragged batch) or null
  int rev = 0;              // LDS-staged scans take their rounds last first
  int nt = 0;               // non-temporal loads (kStreamNtBytes; a template
                            // parameter of the launch)
};

// Moments of pages [split * pages_per_split, ...) of one (b, kv head) for its
// G query heads:
//   mu_p = sum_d (q_d/sqrt(D)) mean_pd (+ ALiBi page-mean bias),
//   sigma_p = sqrt(sum_d (q_d/sqrt(D))^2 std_pd^2),
// and the workgroup's partial sums (of the unbiased mu_p).  A row segment of
// LPR lanes owns a page; U pages per segment in flight.  blockDim == NT.
// Page moments of one workgroup staged in LDS (kLdsOut) before one coalesced
// write-out per head after the scan, when pages_per_split * G fits.  The
// workgroup's partial sums are then formed from LDS in page order, so that
// they do not depend on the order of the scan, which alternates from launch
// to launch (a.rev) like the criticality scan's.
constexpr int kMomentLdsEntries = 4096;

template <typename T, int LPR, int G, int NT, int U, bool kLdsOut = false, bool kNt = false>
__device__ __forceinline__ void moments_partial_block(const MomentsArgs& a, int b, int kvh,
                                                      int split) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SEGS = NT / LPR;
  constexpr int W = NT / 64;
  __shared__ float4 red[G][W];
  __shared__ float2 lds_out[kLdsOut ? kMomentLdsEntries : 1];
  const int seg = threadIdx.x / LPR;
  const int sl = threadIdx.x % LPR;
  const int col = sl * VEC;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int h0 = kvh * G;

  // qs = q / sqrt(D); the variance term is accumulated as (std_d |qs_d|)^2,
  // two operations per element (the product is rounded once more than
  // std_d^2 * qs_d^2, a relative change of 2^-24 per term)
  float qs[G][VEC], qa[G][VEC];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    Vec<T> x;
    x.load((const T*)a.q + b * a.qsb + (h0 + g) * a.qsh + col);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      qs[g][i] = x.v[i] * a.scale;
      qa[g][i] = fabsf(qs[g][i]);
    }
  }
  const T* km = (const T*)a.kmean + b * a.ssb + kvh * a.ssh;
  const T* ks = (const T*)a.kstd + b * a.ssb + kvh * a.ssh;
  // ragged batch: this sequence's own statistics pages, length and position
  int pages = a.pages, stats_len = a.stats_len, q_pos = a.q_pos;
  if (a.seq_lens) {
    const int len = a.seq_lens[b];
    const SeqPages gp = seq_pages(len, a.page_size);
    pages = min(gp.stat_pages, a.pages);
    stats_len = gp.stat_tokens;
    q_pos = len - 1;
  }
  const int p_begin = split * a.pages_per_split;
  const int p_end = min(pages, p_begin + a.pages_per_split);
  float s_mu[G], s_mu2[G], s_var[G], slope[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    s_mu[g] = s_mu2[g] = s_var[g] = 0.f;
    slope[g] = a.slopes ? a.slopes[h0 + g] : 0.f;  // no load inside the scan loop
  }

  // Pages p0 + u * SEGS + seg: unconditional loads (a page past the end
  // re-reads the last one, its result is discarded) so the compiler counts
  // them exactly, in two register buffers: the next round's loads are issued
  // (unconditionally: a conditional prefetch would make every consume wait
  // for it) before the current round's arithmetic.
  constexpr int ROUND = SEGS * U;
  auto fetch = [&](int p0, VecRaw<T> (&mv)[U], VecRaw<T> (&sv)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = min(p0 + u * SEGS + seg, p_end - 1);
      mv[u].load_sel(km + (int64_t)p * a.ssp + col, kNt);
      sv[u].load_sel(ks + (int64_t)p * a.ssp + col, kNt);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the arithmetic
  };
  auto consume = [&](int p0, const VecRaw<T> (&mv)[U], const VecRaw<T> (&sv)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = p0 + u * SEGS + seg;
      const bool ok = p < p_end;
      // a page past the end holds the last page's values (its loads were
      // clamped): its stores rewrite them unchanged, so every lane stores
      // unconditionally and the compiler keeps counting the loads exactly
      const int pc = min(p, p_end - 1);
      const bool acc = ok && sl == 0;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mu = 0.f, var = 0.f;
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          // explicit roundings: both register buffers' inlined copies of this
          // loop give the same bits (the scan order alternates between them)
          const float w = mul_rn(sv[u].get(i), qa[g][i]);
          mu = fma_rn(mv[u].get(i), qs[g][i], mu);
          var = fma_rn(w, w, var);
        }
        mu = seg_sum<LPR>(mu);
        var = seg_sum<LPR>(var);
        if constexpr (!kLdsOut) {
          s_mu[g] += acc ? mu : 0.f;
          s_mu2[g] += acc ? mu * mu : 0.f;
          s_var[g] += acc ? var : 0.f;
        }
        const int64_t o = ((int64_t)b * a.H + h0 + g) * a.pages + pc;
        float mub = mu;
        if (!kLdsOut && a.slopes) {
          // gaussian_utils.py:142-153: slope * (min(p*ps + (ps-1)/2, S'-1) - q_pos)
          const float pos = fminf((float)pc * (float)a.page_size + (float)(a.page_size - 1) * 0.5f,
                                  (float)(stats_len - 1));
          mub = add_rn(mu, mul_rn(slope[g], sub_rn(pos, (float)q_pos)));
        }
        if constexpr (kLdsOut) {
          // the raw moments; the bias, the root and the sums come after the scan
          if (sl == 0) lds_out[(pc - p_begin) * G + g] = make_float2(mu, var);
        } else {
          a.mu_p[o] = mub;
          a.sigma_p[o] = sqrtf(var);
        }
      }
    }
  };
  if (p_begin < p_end) {
    // round k of nr starts at page start(k); reversed, the last round first
    // (a round past either end re-reads clamped pages and discards them)
    const int nr = (p_end - p_begin + ROUND - 1) / ROUND;
    const bool rev = kLdsOut && a.rev;
    auto start = [&](int k) { return p_begin + (rev ? nr - 1 - k : k) * ROUND; };
    VecRaw<T> mv_a[U], sv_a[U], mv_b[U], sv_b[U];
    fetch(start(0), mv_a, sv_a);
    for (int k = 0; k < nr; k += 2) {
      fetch(k + 1 < nr ? start(k + 1) : p_end, mv_b, sv_b);
      consume(start(k), mv_a, sv_a);
      if (k + 1 >= nr) break;
      fetch(k + 2 < nr ? start(k + 2) : p_end, mv_a, sv_a);
      consume(start(k + 1), mv_b, sv_b);
    }
  }
  if constexpr (kLdsOut) {
    // page moments out (with the ALiBi page-mean bias and the root), and the
    // partial sums of the unbiased mu_p in page order, thread j taking pages
    // j, j + NT, ...
    __syncthreads();
    const int np = max(p_end - p_begin, 0);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t o = ((int64_t)b * a.H + h0 + g) * a.pages + p_begin;
      for (int j = threadIdx.x; j < np; j += NT) {
        const float2 v = lds_out[j * G + g];
        float mub = v.x;
        if (a.slopes) {
          // gaussian_utils.py:142-153: slope * (min(p*ps + (ps-1)/2, S'-1) - q_pos)
          const float pos = fminf((float)(p_begin + j) * (float)a.page_size +
                                      (float)(a.page_size - 1) * 0.5f,
                                  (float)(stats_len - 1));
          mub = add_rn(v.x, mul_rn(slope[g], sub_rn(pos, (float)q_pos)));
        }
        a.mu_p[o + j] = mub;
        a.sigma_p[o + j] = sqrtf(v.y);
        s_mu[g] += v.x;
        s_mu2[g] += v.x * v.x;
        s_var[g] += v.y;
      }
    }
  }
  // workgroup partials in a fixed order: lanes, then waves
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float x = wave_sum(s_mu[g]), y = wave_sum(s_mu2[g]), z = wave_sum(s_var[g]);
    if (lane == 0) red[g][wid] = make_float4(x, y, z, 0.f);
  }
  __syncthreads();
  if (threadIdx.x < G) {
    const int g = threadIdx.x;
    float4 r = red[g][0];
#pragma unroll
    for (int w = 1; w < W; ++w) {
      r.x += red[g][w].x;
      r.y += red[g][w].y;
      r.z += red[g][w].z;
    }
    a.partials[((int64_t)b * a.H + h0 + g) * a.splits + split] = r;
  }
}

// Sum of one head's `splits` partials held by an aligned segment of
// S2 = split_lanes(splits) lanes (lane j of the segment holds partial j, the
// lanes past `splits` hold zeros); every lane of the segment receives the
// sum.  The lane-tree order is fixed, so every consumer of a head's partials
// (the standalone finalize launch and the fused step) derives the same bits.
__host__ __device__ __forceinline__ int split_lanes(int splits) {
  int s2 = 1;
  while (s2 < splits) s2 *= 2;
  return s2;
}

template <int L>
__device__ __forceinline__ float4 seg_sum4(float4 x) {
  return make_float4(seg_sum<L>(x.x), seg_sum<L>(x.y), seg_sum<L>(x.z), 0.f);
}

__device__ __forceinline__ float4 reduce_splits(float4 x, int s2) {
  switch (s2) {
    case 1: return x;
    case 2: return seg_sum4<2>(x);
    case 4: return seg_sum4<4>(x);
    case 8: return seg_sum4<8>(x);
    case 16: return seg_sum4<16>(x);
    case 32: return seg_sum4<32>(x);
    default: return seg_sum4<64>(x);
  }
}

struct Moments {
  float mu_g, sigma_g, mean_var, var_means;
};

// Global moments of a head from its sums over `pages` pages: mean of mu_p,
// sigma_g = sqrt(mean sigma_p^2 + population variance of mu_p), with the
// reference's nan/inf clean-up and clamp (gaussian_utils.py:155-161).
__device__ __forceinline__ Moments finalize_moments(float4 s, int pages) {
  const float denom = (float)pages;
  const float mean = s.x / denom;
  const float mvar = s.z / denom;
  const float vmeans = fmaxf(s.y / denom - mean * mean, 0.0f);
  float sg = sqrtf(mvar + vmeans);
  if (sg != sg) sg = 1e-6f;
  else if (isinf(sg)) sg = sg > 0 ? 1e6f : 1e-6f;
  sg = fmaxf(sg, 1e-6f);
  float mg = mean;
  if (mg != mg || isinf(mg)) mg = 0.f;
  return Moments{mg, sg, mvar, vmeans};
}

// ---------------------------------------------------------------------------
// threshold selection + pack + clamp + compacted lengths of one (b, kv head)
// ---------------------------------------------------------------------------

struct SelectArgs {
  const float* mu_p;
  const float* sigma_p;
  int B, H, Hkv;
  int pages;      // pages_for_stats
  int num_pages;  // pages incl. the in-progress last page
  float am1;
  int auto_margins;
  float smz;                      // used when !auto_margins
  float z_page;                   // used when !auto_margins
  float z_page_low, z_page_high;  // auto: max_quantile 0.99 / 0.995
  float frac;
  int32_t* page_indices;
  int64_t pisb, pish;
  int32_t* counts;         // [B, Hkv]
  float* tau_floor;        // [B, H]
  int32_t* cache_seqlens;  // [B, Hkv] or null
  int page_size;
  int last_page_size;
  float* tau_clamped;      // [B, H] or null
  float z_clamp;
  float eps;
  float* eff;              // [2] = (safety_margin_z, max_quantile) or null
  const int32_t* seq_lens; // [B] per-sequence lengths (ragged batch) or null; `pages`
                           // and `num_pages` are then the longest sequence's
};

// Per-head scalars of the single-Gaussian tau-hat for batch element b: the
// statistics pages, n = seq_len_for_stats and sqrt(2 ln(n + 1)).
struct TauGeom {
  int pages;
  float n, lnf;
};
__device__ __forceinline__ TauGeom tau_geom(const int32_t* seq_lens, int b, int ps, int pages,
                                            float n, float lnf) {
  TauGeom t{pages, n, lnf};
  if (seq_lens) {
    const SeqPages gp = seq_pages(seq_lens[b], ps);
    t.pages = gp.stat_pages;
    t.n = (float)gp.stat_tokens;
    t.lnf = (float)sqrt(2.0 * log((double)gp.stat_tokens + 1.0));
  }
  return t;
}

// Selects the pages of one (b, kv head) given each query head's tau-hat
// (`tau_hat[g]`), sigma_g (`sig_g[g]`) and the batch-wide mean sigma_g
// (`sbar`, used with automatic margins).  Writes the ascending page table
// (+ the last page as sentinel) to global memory and, for slots < lds_cap, to
// `lds_pages`; the count, tau floor, compacted length and (with clamp) the
// clamped tau, which is also returned in tau_out[g] (tau-hat when not
// clamping).  `upper_in[g]`, when given, is the head's mean of
// mu_p + 1.5 sigma_p over the pages (else computed here).  Returns the page
// count.  blockDim == NT; every thread returns the same count.
//
// Pack: each wave owns a contiguous range of pages; one pass counts its
// selected pages (ballots), one barrier publishes the counts, a second pass
// writes them at their ranks.  Selected page ids therefore come out ascending.
template <int G, int NT>
__device__ __forceinline__ int select_pack_block(const SelectArgs& a, int b, int kvh, float sbar,
                                                 const float* tau_hat, const float* sig_g,
                                                 int* lds_pages, int lds_cap, float* tau_out,
                                                 const float* upper_in = nullptr) {
  constexpr int W = NT / 64;
  __shared__ float scratch[16];
  __shared__ int wave_cnt[W];
  __shared__ float cm[G][W];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int bkv = b * a.Hkv + kvh;
  const int h0 = kvh * G;
  // this sequence's pages (ragged batch) within rows of stride a.pages
  int pages = a.pages, num_pages = a.num_pages, last_page_size = a.last_page_size;
  if (a.seq_lens) {
    const SeqPages gp = seq_pages(a.seq_lens[b], a.page_size);
    pages = min(gp.stat_pages, a.pages);
    num_pages = min(gp.pages, a.num_pages);
    last_page_size = gp.last_size;
  }

  float smz = a.smz, z_page = a.z_page;
  if (a.auto_margins) {
    const bool low = sbar < 1.5f;
    smz = (float)((low ? 0.01 : 0.05) * (double)sbar);
    z_page = low ? a.z_page_low : a.z_page_high;
    if (bkv == 0 && tid == 0 && a.eff) {
      a.eff[0] = smz;
      a.eff[1] = low ? 0.99f : 0.995f;
    }
  }

  float tfloor[G];
  const float* mu[G];
  const float* sg[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int h = h0 + g;
    mu[g] = a.mu_p + ((int64_t)b * a.H + h) * a.pages;
    sg[g] = a.sigma_p + ((int64_t)b * a.H + h) * a.pages;
    float upper;
    if (upper_in) {
      upper = upper_in[g];
    } else {
      float s = 0.f;
      for (int p = tid; p < pages; p += NT) s += fma_rn(1.5f, sg[g][p], mu[g][p]);
      upper = block_sum(s, scratch) / (float)pages;
    }
    const float th = tau_hat[g];
    const float thr = th / a.am1;
    const float sig_delta = smz * sig_g[g];
    const float excess = fmaxf(thr - upper, 0.0f);
    const float tau_delta = a.frac * excess;
    const float delta = fmaxf(sig_delta, tau_delta);
    tfloor[g] = fma_rn(-delta, a.am1, th);
    if (tid == 0) a.tau_floor[b * a.H + h] = tfloor[g];
  }

  // page p is selected when any query head of the group selects it
  auto selected = [&](int p) {
    bool sel = false;
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (mul_rn(a.am1, fma_rn(z_page, sg[g][p], mu[g][p])) > tfloor[g]) sel = true;
    return sel;
  };
  const float third = 0.3333333333333333f;
  float capmax[G];
#pragma unroll
  for (int g = 0; g < G; ++g) capmax[g] = -INFINITY;
  const int per = (pages + W - 1) / W;
  const int pw0 = min(pages, wid * per), pw1 = min(pages, pw0 + per);
  // kSelBatch rounds of 64 pages per wave at a time: their loads are issued
  // together (clamped to the wave's last page, unconditional), so a wave
  // waits once per batch instead of once per round
  constexpr int kSelBatch = 4;
  int cnt = 0;
  for (int r0 = pw0; r0 < pw1; r0 += 64 * kSelBatch) {
    float mv[kSelBatch][G], sv[kSelBatch][G];
#pragma unroll
    for (int u = 0; u < kSelBatch; ++u) {
      const int pc = min(r0 + u * 64 + lane, pw1 - 1);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        mv[u][g] = mu[g][pc];
        sv[u][g] = sg[g][pc];
      }
    }
#pragma unroll
    for (int u = 0; u < kSelBatch; ++u) {
      bool sel = false;
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (mul_rn(a.am1, fma_rn(z_page, sv[u][g], mv[u][g])) > tfloor[g]) sel = true;
      sel = sel && r0 + u * 64 + lane < pw1;
      if (sel) {
#pragma unroll
        for (int g = 0; g < G; ++g)
          capmax[g] = fmaxf(capmax[g], fma_rn(mul_rn(a.z_clamp, sv[u][g]), third, mv[u][g]));
      }
      cnt += __popcll(__ballot(sel));
    }
  }
  if (lane == 0) wave_cnt[wid] = cnt;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float m = wave_max(capmax[g]);
    if (lane == 0) cm[g][wid] = m;
  }
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const int c = wave_cnt[w];
    base += w < wid ? c : 0;
    total += c;
  }
  int32_t* out = a.page_indices + b * a.pisb + kvh * a.pish;
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
  for (int r0 = pw0; r0 < pw1; r0 += 64 * kSelBatch) {
    bool selb[kSelBatch];
#pragma unroll
    for (int u = 0; u < kSelBatch; ++u) selb[u] = selected(min(r0 + u * 64 + lane, pw1 - 1));
#pragma unroll
    for (int u = 0; u < kSelBatch; ++u) {
      const int p = r0 + u * 64 + lane;
      const bool sel = selb[u] && p < pw1;
      const uint64_t m = __ballot(sel);
      if (sel) {
        const int slot = base + __popcll(m & below);
        out[slot] = p;
        if (slot < lds_cap) lds_pages[slot] = p;
      }
      base += __popcll(m);
    }
  }
  int count = total;
  if (num_pages > pages) {
    if (tid == 0) {
      out[total] = num_pages - 1;
      if (total < lds_cap) lds_pages[total] = num_pages - 1;
    }
    count = total + 1;
  }
  if (tid == 0) {
    a.counts[bkv] = count;
    if (a.cache_seqlens) a.cache_seqlens[bkv] = max(count - 1, 0) * a.page_size + last_page_size;
  }
  // clamp: tau = min(tau_hat, max((alpha-1) * max cap over the selection - eps, floor))
#pragma unroll
  for (int g = 0; g < G; ++g) {
    if (tid == g) {
      const float th = tau_hat[g];
      float tc = th;
      if (a.tau_clamped) {
        float mx = -INFINITY;
        for (int w = 0; w < W; ++w) mx = fmaxf(mx, cm[g][w]);
        const float up = fmaxf(fma_rn(a.am1, mx, -a.eps), tfloor[g]);
        tc = (mx > -3.0e38f) ? fminf(th, up) : th;
        a.tau_clamped[b * a.H + h0 + g] = tc;
      }
      if (tau_out) tau_out[g] = tc;
    }
  }
  return count;
}

}  // namespace gauss
}  // namespace ekv
