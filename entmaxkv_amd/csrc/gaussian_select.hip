// Gaussian-aware page selection: page score moments, the tau-hat solvers,
// threshold selection + pack, tau clamp and compacted lengths.
//
//   gaussian_stats_kernel   kernels/gaussian_page_stats.py:8-121 and
//                           gaussian_utils.py:130-181: per page
//                           mu_p = sum_d (q_d/sqrt(D)) kmean_pd,
//                           var_p = sum_d (q_d/sqrt(D))^2 kstd_pd^2, global
//                           moments per head and (fused, last workgroup per
//                           (b, kv head)) the single-Gaussian tau-hat solve.
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
#include "ekv_common.h"
#include "../../include/entmaxkv.h"

using namespace ekv;

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

__device__ __forceinline__ float normal_pdf(float x) {
  return expf(-0.5f * x * x) * 0.3989422804014327f;
}
// Phi(x) = 0.5 * erfc(-x / sqrt(2)): equal to 0.5 * (1 + erf(x / sqrt(2))) but
// without the cancellation of 1 + erf in the lower tail.
__device__ __forceinline__ float normal_cdf(float x) {
  return 0.5f * erfcf(-x * 0.7071067811865476f);
}

// f(tau) = n*E[[(alpha-1)S - tau]_+^(1/(alpha-1))] - 1 for S ~ N(mu, sigma^2)
// (count weight `n`), with first and second derivatives.  The third moment
// used for alpha = 4/3 is the reference's expression (tau_solver.py:104-107).
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

// Bracketed Halley solve of one single-Gaussian problem (one lane).  The
// iteration rule is the reference's; it stops early once a candidate is
// accepted (|f| <= tol) after a step below 1e-6 * max(1, |tau|), which leaves
// tau within the tolerance band the remaining fixed-count steps would keep it in.
__device__ float solve_single_gaussian(float mu, float sigma, float n, float alpha, float log_n_factor,
                                       int iterations, float tol) {
  sigma = fmaxf(sigma, 1.0e-6f);
  const float a = alpha - 1.0f;
  const float radius = a * sigma * (log_n_factor + 8.0f);
  float lo = a * mu - radius, hi = a * mu + radius;
  float t = 0.5f * (lo + hi);
  for (int it = 0; it < iterations; ++it) {
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
      if (small) break;
    } else {
      t = 0.5f * (lo + hi);
    }
  }
  return t;
}

// ---------------------------------------------------------------------------
// per-page score moments (+ fused global moments and tau-hat)
// ---------------------------------------------------------------------------

struct StatsArgs {
  const void* q;
  int64_t qsb, qsh;
  const void* kmean;
  const void* kstd;
  int64_t ssb, ssh, ssp;
  int pages;  // pages_for_stats
  int H, Hkv;
  float scale;  // 1/sqrt(D) in fp32
  const float* slopes;
  int page_size;
  int q_pos;        // seq_len - 1
  int stats_len;    // seq_len_for_stats
  float* mu_p;      // [B, H, pages]
  float* sigma_p;   // [B, H, pages]
  float* mu_g;      // [B, H]
  float* sigma_g;
  float* mean_var;
  float* var_means;
  float* tau_hat;   // [B, H] or null
  float alpha;
  float n_tokens;
  float log_n_factor;
  int tau_iters;
  float tol;
  float* ws_tiles;  // [B, H, tiles, 3]
  int* counters;    // [B, Hkv]
};

template <typename T, int LPR, int G>
__global__ __launch_bounds__(kThreads) void gaussian_stats_kernel(StatsArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SEGS = kThreads / LPR;
  __shared__ float red[3][G][SEGS * kUnroll];
  const int seg = threadIdx.x / LPR;
  const int sl = threadIdx.x % LPR;
  const int col = sl * VEC;
  const int bkv = blockIdx.y;
  const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
  const int h0 = kvh * G;

  float qs[G][VEC], qq[G][VEC];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    Vec<T> x;
    x.load((const T*)a.q + b * a.qsb + (h0 + g) * a.qsh + col);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      qs[g][i] = x.v[i] * a.scale;
      qq[g][i] = qs[g][i] * qs[g][i];
    }
  }
  const T* km = (const T*)a.kmean + b * a.ssb + kvh * a.ssh;
  const T* ks = (const T*)a.kstd + b * a.ssb + kvh * a.ssh;
  const int p_base = blockIdx.x * (SEGS * kUnroll) + seg;
  VecRaw<T> mv[kUnroll], sv[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int p = p_base + u * SEGS;
    if (p < a.pages) {
      mv[u].load(km + (int64_t)p * a.ssp + col);
      sv[u].load(ks + (int64_t)p * a.ssp + col);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int p = p_base + u * SEGS;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mu = 0.f, var = 0.f;
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float sd = sv[u].get(i);
        mu += mv[u].get(i) * qs[g][i];
        var += (sd * sd) * qq[g][i];
      }
      mu = seg_sum<LPR>(mu);
      var = seg_sum<LPR>(var);
      if (sl == 0) {
        const bool ok = p < a.pages;
        red[0][g][u * SEGS + seg] = ok ? mu : 0.f;
        red[1][g][u * SEGS + seg] = ok ? mu * mu : 0.f;
        red[2][g][u * SEGS + seg] = ok ? var : 0.f;
        if (ok) {
          const int64_t o = ((int64_t)b * a.H + h0 + g) * a.pages + p;
          float mub = mu;
          if (a.slopes) {
            // gaussian_utils.py:142-153: slope * (min(p*ps + (ps-1)/2, S'-1) - q_pos)
            const float pos = fminf((float)p * (float)a.page_size + (float)(a.page_size - 1) * 0.5f,
                                    (float)(a.stats_len - 1));
            mub = add_rn(mu, mul_rn(a.slopes[h0 + g], sub_rn(pos, (float)a.q_pos)));
          }
          a.mu_p[o] = mub;
          a.sigma_p[o] = sqrtf(var);
        }
      }
    }
  }
  __syncthreads();
  // tile partial sums (deterministic order), one wave per (quantity, head)
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int j = wid; j < 3 * G; j += kThreads / 64) {
    const int qn = j / G, g = j % G;
    float x = 0.f;
    for (int r = lane; r < SEGS * kUnroll; r += 64) x += red[qn][g][r];
    x = wave_sum(x);
    if (lane == 0)
      st_coherent(a.ws_tiles + (((int64_t)b * a.H + h0 + g) * gridDim.x + blockIdx.x) * 3 + qn, x);
  }
  if (!last_arrival(&a.counters[bkv], gridDim.x)) return;

  for (int g = wid; g < G; g += kThreads / 64) {
    const int h = h0 + g;
    const float* tl = a.ws_tiles + ((int64_t)b * a.H + h) * gridDim.x * 3;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f;
    for (int t = lane; t < (int)gridDim.x; t += 64) {
      s0 += ld_coherent(tl + t * 3 + 0);
      s1 += ld_coherent(tl + t * 3 + 1);
      s2 += ld_coherent(tl + t * 3 + 2);
    }
    s0 = wave_sum(s0);
    s1 = wave_sum(s1);
    s2 = wave_sum(s2);
    if (lane == 0) {
      const float denom = (float)a.pages;
      const float mean = s0 / denom;
      const float mvar = s2 / denom;
      const float vmeans = fmaxf(s1 / denom - mean * mean, 0.0f);
      float sg = sqrtf(mvar + vmeans);
      if (sg != sg) sg = 1e-6f;
      else if (isinf(sg)) sg = sg > 0 ? 1e6f : 1e-6f;
      sg = fmaxf(sg, 1e-6f);
      float mg = mean;
      if (mg != mg || isinf(mg)) mg = 0.f;
      const int o = b * a.H + h;
      a.mu_g[o] = mg;
      a.sigma_g[o] = sg;
      a.mean_var[o] = mvar;
      a.var_means[o] = vmeans;
      if (a.tau_hat)
        a.tau_hat[o] = solve_single_gaussian(mg, sg, a.n_tokens, a.alpha, a.log_n_factor,
                                             a.tau_iters, a.tol);
    }
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
                                                               float* out, int pages, float cnt,
                                                               float alpha, int iters, float tol) {
  __shared__ float scratch[16];
  const int row = blockIdx.x;
  const float* mu = mu_p + (int64_t)row * pages;
  const float* sg = sigma_p + (int64_t)row * pages;
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

struct SelectArgs {
  const float* mu_p;
  const float* sigma_p;
  const float* tau_hat;
  const float* sigma_g;
  int B, H, Hkv;
  int pages;      // pages_for_stats
  int num_pages;  // pages incl. the in-progress last page
  float am1;
  int auto_margins;
  float smz;        // used when !auto_margins
  float z_page;     // used when !auto_margins
  float z_page_low, z_page_high;  // auto: max_quantile 0.99 / 0.995
  float frac;
  int32_t* page_indices;
  int64_t pisb, pish;
  int32_t* counts;  // [B, Hkv]
  float* tau_floor; // [B, H]
  int32_t* cache_seqlens;  // [B, Hkv] or null
  int page_size;
  int last_page_size;
  float* tau_clamped;  // [B, H] or null
  float z_clamp;
  float eps;
  float* eff;  // [2] = (safety_margin_z, max_quantile) or null
};

template <int G>
__global__ __launch_bounds__(kThreads) void select_pack_kernel(SelectArgs a) {
  __shared__ float scratch[16];
  __shared__ int scan_scratch[kThreads / 64 + 1];
  const int tid = threadIdx.x;
  const int bkv = blockIdx.x;
  const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
  const int h0 = kvh * G;

  float smz = a.smz, z_page = a.z_page;
  if (a.auto_margins) {
    float s = 0.f;
    const int nh = a.B * a.H;
    for (int i = tid; i < nh; i += kThreads) s += a.sigma_g[i];
    const float sbar = block_sum(s, scratch) / (float)nh;
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
    float s = 0.f;
    for (int p = tid; p < a.pages; p += kThreads) s += fma_rn(1.5f, sg[g][p], mu[g][p]);
    const float upper = block_sum(s, scratch) / (float)a.pages;
    const float th = a.tau_hat[b * a.H + h];
    const float thr = th / a.am1;
    const float sig_delta = smz * a.sigma_g[b * a.H + h];
    const float excess = fmaxf(thr - upper, 0.0f);
    const float tau_delta = a.frac * excess;
    const float delta = fmaxf(sig_delta, tau_delta);
    tfloor[g] = fma_rn(-delta, a.am1, th);
    if (tid == 0) a.tau_floor[b * a.H + h] = tfloor[g];
  }

  const float third = 0.3333333333333333f;
  float capmax[G];
#pragma unroll
  for (int g = 0; g < G; ++g) capmax[g] = -INFINITY;
  int32_t* out = a.page_indices + b * a.pisb + kvh * a.pish;
  int base = 0;
  for (int c0 = 0; c0 < a.pages; c0 += kThreads) {
    const int p = c0 + tid;
    bool sel = false;
    if (p < a.pages) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float m = mu[g][p], s = sg[g][p];
        if (mul_rn(a.am1, fma_rn(z_page, s, m)) > tfloor[g]) sel = true;
      }
      if (sel) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float cap = fma_rn(mul_rn(a.z_clamp, sg[g][p]), third, mu[g][p]);
          capmax[g] = fmaxf(capmax[g], cap);
        }
      }
    }
    int tot;
    const int pos = block_excl_scan(sel ? 1 : 0, scan_scratch, &tot);
    if (sel) out[base + pos] = p;
    base += tot;
  }
  int count = base;
  if (a.num_pages > a.pages) {
    if (tid == 0) out[base] = a.num_pages - 1;
    count = base + 1;
  }
  if (tid == 0) {
    a.counts[bkv] = count;
    if (a.cache_seqlens) a.cache_seqlens[bkv] = max(count - 1, 0) * a.page_size + a.last_page_size;
  }
  if (a.tau_clamped) {
    // block max of each head's cap over the selected pages
    __shared__ float cm[kThreads / 64];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float m = wave_max(capmax[g]);
      if ((tid & 63) == 0) cm[tid >> 6] = m;
      __syncthreads();
      if (tid == 0) {
        float mx = -INFINITY;
        for (int w = 0; w < kThreads / 64; ++w) mx = fmaxf(mx, cm[w]);
        const int h = h0 + g;
        const float th = a.tau_hat[b * a.H + h];
        float up = fmaxf(fma_rn(a.am1, mx, -a.eps), tfloor[g]);
        a.tau_clamped[b * a.H + h] = (mx > -3.0e38f) ? fminf(th, up) : th;
      }
      __syncthreads();
    }
  }
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

extern "C" int64_t ekv_gaussian_workspace_bytes(int B, int H, int Hkv, int D, int pages, int dtype) {
  const int lpr = D / (dtype == kF32 ? 4 : 8);
  const int ppw = lpr > 0 ? (kThreads / lpr) * kUnroll : 1;
  const int64_t tiles = (pages + ppw - 1) / ppw;
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  return up((int64_t)B * Hkv * 4) + up((int64_t)B * H * tiles * 3 * 4);
}

extern "C" int ekv_gaussian_page_stats(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kmean, const void* kstd,
    int64_t s_stride_b, int64_t s_stride_h, int64_t s_stride_page, int pages_for_stats,
    const float* alibi_slopes, int page_size, int seq_len, float* mu_p, float* sigma_p, float* mu_g,
    float* sigma_g, float* mean_var, float* var_means, float* tau_hat, float alpha, int n_tokens,
    int tau_iters, float tol, int B, int H, int Hkv, int D, void* workspace,
    int64_t workspace_bytes, int dtype, void* stream) {
  EKV_REQUIRE(q && kmean && kstd && mu_p && sigma_p && mu_g && sigma_g && mean_var && var_means &&
                  workspace,
              "ekv_gaussian_page_stats: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "ekv_gaussian_page_stats: bad heads");
  EKV_REQUIRE(pages_for_stats > 0, "ekv_gaussian_page_stats: pages_for_stats must be positive");
  EKV_REQUIRE(!tau_hat || alpha == 2.0f || alpha == 1.5f || fabsf(alpha - 4.0f / 3.0f) < 1e-6f,
              "ekv_gaussian_page_stats: tau-hat needs alpha in {2, 1.5, 4/3}");
  EKV_REQUIRE(workspace_bytes >= ekv_gaussian_workspace_bytes(B, H, Hkv, D, pages_for_stats, dtype),
              "ekv_gaussian_page_stats: workspace too small");
  StatsArgs a;
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  a.counters = (int*)workspace;
  a.ws_tiles = (float*)((char*)workspace + up((int64_t)B * Hkv * 4));
  a.q = q;
  a.qsb = q_stride_b;
  a.qsh = q_stride_h;
  a.kmean = kmean;
  a.kstd = kstd;
  a.ssb = s_stride_b;
  a.ssh = s_stride_h;
  a.ssp = s_stride_page;
  a.pages = pages_for_stats;
  a.H = H;
  a.Hkv = Hkv;
  a.scale = (float)(1.0 / sqrt((double)D));
  a.slopes = alibi_slopes;
  a.page_size = page_size;
  a.q_pos = seq_len - 1;
  a.stats_len = n_tokens;
  a.mu_p = mu_p;
  a.sigma_p = sigma_p;
  a.mu_g = mu_g;
  a.sigma_g = sigma_g;
  a.mean_var = mean_var;
  a.var_means = var_means;
  a.tau_hat = tau_hat;
  a.alpha = fabsf(alpha - 4.0f / 3.0f) < 1e-6f ? 4.0f / 3.0f : alpha;
  a.n_tokens = (float)n_tokens;
  a.log_n_factor = (float)sqrt(2.0 * log((double)n_tokens + 1.0));
  a.tau_iters = tau_iters;
  a.tol = tol;
  hipStream_t s = (hipStream_t)stream;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    return dispatch_lpr<T>(D, [&](auto lpr) {
      constexpr int LPR = decltype(lpr)::value;
      return dispatch_group(H / Hkv, [&](auto gv) {
        constexpr int G = decltype(gv)::value;
        constexpr int PPW = (kThreads / LPR) * kUnroll;
        dim3 grid((pages_for_stats + PPW - 1) / PPW, B * Hkv);
        hipLaunchKernelGGL((gaussian_stats_kernel<T, LPR, G>), grid, dim3(kThreads), 0, s, a);
        return check_launch("gaussian_stats_kernel");
      });
    });
  });
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
                                    float tol, void* stream) {
  EKV_REQUIRE(mu_p && sigma_p && tau_out && rows >= 0 && pages > 0 && page_count > 0.f,
              "ekv_tau_page_mixture: bad arguments");
  if (rows == 0) return EKV_OK;
  hipLaunchKernelGGL(tau_mixture_kernel, dim3(rows), dim3(kThreads), 0, (hipStream_t)stream, mu_p,
                     sigma_p, tau_out, pages, page_count, alpha, max_iter, tol);
  return check_launch("tau_mixture_kernel");
}

extern "C" int ekv_select_gaussian_pack(
    const float* mu_p, const float* sigma_p, const float* tau_hat, const float* sigma_g, int B,
    int H, int Hkv, int pages_for_stats, int num_pages, float alpha, int auto_margins,
    float safety_margin_z, float z_page, float z_page_low, float z_page_high,
    float threshold_excess_margin_fraction, int32_t* page_indices, int64_t pi_stride_b,
    int64_t pi_stride_h, int32_t* counts, float* tau_floor, int32_t* cache_seqlens, int page_size,
    int last_page_size, float* tau_clamped, float z_clamp, float eps, float* effective_margins,
    void* stream) {
  EKV_REQUIRE(mu_p && sigma_p && tau_hat && sigma_g && page_indices && counts && tau_floor,
              "ekv_select_gaussian_pack: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "ekv_select_gaussian_pack: bad heads");
  EKV_REQUIRE(pages_for_stats > 0 && num_pages >= pages_for_stats,
              "ekv_select_gaussian_pack: pages_for_stats and num_pages must be positive");
  SelectArgs a;
  a.mu_p = mu_p;
  a.sigma_p = sigma_p;
  a.tau_hat = tau_hat;
  a.sigma_g = sigma_g;
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
  hipStream_t s = (hipStream_t)stream;
  return dispatch_group(H / Hkv, [&](auto gv) {
    constexpr int G = decltype(gv)::value;
    hipLaunchKernelGGL((select_pack_kernel<G>), dim3(B * Hkv), dim3(kThreads), 0, s, a);
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
