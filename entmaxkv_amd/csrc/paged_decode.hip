// Paged split-KV alpha-entmax decode over a compacted page table.
//
// Follows kernels/adadecode_paged.py:567-762 (exact tau: global max,
// 16-bin histogram init, bracketed Halley, output) and
// kernels/adadecode_paged_gaussian_tau.py:192-331 (given tau: unbounded
// Halley/Newton corrections, output).  Compacted token c of (b, kv head) lives
// in cache row page_indices[c / ps] * ps + c % ps; scores are
// s_c = qs . k_c with qs = q * (alpha-1)/sqrt(D) rounded to the input dtype,
// the output is out = sum_c [s_c - tau]_+^(1/(alpha-1)) v_c (not renormalised,
// as in the reference).
//
// Two kernels instead of the reference's 7 + 2*niter launches:
//   score_tau_kernel  grid (splits, B*Hkv): each workgroup streams its share
//     of the selected K rows once (16-byte loads, all G query heads of the
//     group served by one load) and writes fp32 scores to the workspace; the
//     last workgroup of a (b, kv head) solves tau for the group's heads over
//     the L2-resident scores, one wave per head.
//   weighted_sum_kernel  grid (splits, B*Hkv): each workgroup re-reads its
//     scores, compacts the tokens with s > tau (the entmax support), gathers
//     only those V rows, and writes a per-split fp32 partial; the last
//     workgroup sums the partials in split order (deterministic, no atomics)
//     and writes out in the input dtype.
// K is read once and V only on the support; the reference reads K 3+niter
// times.
#include "ekv_common.h"
#include "../../include/entmaxkv.h"

using namespace ekv;

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;
constexpr int kBins = 16;

struct DecodeArgs {
  const void* q;
  int64_t qsb, qsh;
  const void* k;
  const void* v;
  int64_t ksb, ksh, ksr;
  int64_t row_limit;  // rows addressable in each (b, kv head) of K/V
  const int32_t* page_indices;
  int64_t pisb, pish;
  int n_slots;
  const int32_t* cache_seqlens;
  int64_t csb, csh;
  const int32_t* q_seqlens;
  const float* slopes;
  float* tau;  // [B, H]
  int tau_mode;  // 0 exact (histogram + bracketed Halley), 1 given tau (unbounded Halley)
  int iters;
  void* out;
  int64_t osb, osh;
  float alpha;
  float qscale;  // (alpha-1)/sqrt(D) already rounded to the input dtype
  int page_size;
  int H, Hkv;
  int splits;
  int max_tokens;
  float* ws_scores;   // [B, H, max_tokens]
  float* ws_partial;  // [B, H, splits, D]
  int* ws_flags;      // [B, Hkv, splits]
  int* counters;      // [2, B, Hkv]
};

__device__ __forceinline__ int token_count(const DecodeArgs& a, int b, int kvh) {
  int n = a.cache_seqlens[b * a.csb + kvh * a.csh];
  n = max(n, 0);
  return min(n, min(a.n_slots * a.page_size, a.max_tokens));
}

// Maps compacted token c to its cache row, or -1 when the page id is outside
// the cache (a malformed table never causes an out-of-bounds access).
__device__ __forceinline__ int64_t token_row(const int32_t* __restrict__ pi, int c, int ps,
                                             int64_t row_limit) {
  const int page = pi[c / ps];
  const int64_t row = (int64_t)page * ps + (c % ps);
  return (page >= 0 && row < row_limit) ? row : -1;
}

// entmax weight of an active score difference x > 0
__device__ __forceinline__ float entmax_weight(float x, float alpha, float c0) {
  if (alpha == 2.0f) return x;
  if (alpha == 1.5f) return x * x;
  return exp2f(log2f(x) * c0);
}

// ---------------------------------------------------------------------------
// tau solve for one head, executed by one full wave over L2-resident scores
// ---------------------------------------------------------------------------

__device__ __forceinline__ void accumulate(const float* __restrict__ sc, int n, float t, float alpha,
                                           float c0, float& a0, float& a1, float& a2) {
  const int lane = threadIdx.x & 63;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f;
  for (int c = lane; c < n; c += 64) {
    const float x = sc[c];
    if (x > t) {
      const float d = x - t;
      if (alpha == 2.0f) {
        s0 += d;
        s1 += 1.f;
      } else if (alpha == 1.5f) {
        s0 += d * d;
        s1 += d;
        s2 += 1.f;
      } else {
        const float l = log2f(d);
        s0 += exp2f(l * c0);
        s1 += exp2f(l * (c0 - 1.f));
        s2 += exp2f(l * (c0 - 2.f));
      }
    }
  }
  a0 = wave_sum(s0);
  a1 = wave_sum(s1);
  a2 = wave_sum(s2);
}

// kernels/adadecode.py:38-112 (alpha 2, 1.5 and generic bin search)
__device__ void histogram_init(const int* hist, float gmax, float alpha, float& t, float& t_lo,
                               float& t_hi) {
  const float t0 = gmax - 1.0f;
  if (alpha == 2.0f || alpha == 1.5f) {
    float sum_z = 1.f, sum_k = 1.f, sum_z2 = 1.f;
    for (int sj = kBins - 1; sj >= 0; --sj) {
      float c_bin = (float)hist[sj];
      if (sj == kBins - 1) c_bin -= 1.0f;
      const float c_tau = (float)sj / (float)kBins;
      const float new_z = sum_z + c_bin * c_tau;
      const float new_k = sum_k + c_bin;
      if (alpha == 2.0f) {
        if ((new_z - new_k * c_tau) < 1.0f) {
          sum_z = new_z;
          sum_k = new_k;
        }
      } else {
        const float new_z2 = sum_z2 + c_bin * (c_tau * c_tau);
        if (new_k * c_tau * c_tau - 2.0f * new_z * c_tau + new_z2 < 1.0f) {
          sum_z = new_z;
          sum_k = new_k;
          sum_z2 = new_z2;
        }
      }
    }
    float t_init;
    if (alpha == 2.0f) {
      t_init = gmax + (sum_z - 1.0f) / sum_k - 1.0f;
    } else {
      const float disc = sum_z * sum_z - sum_k * (sum_z2 - 1.0f);
      t_init = gmax + (sum_z - sqrtf(disc)) / sum_k - 1.0f;
    }
    t_lo = t_init;
    t_hi = t_init + 1.0f / kBins;
  } else {
    const float p = 1.0f / (alpha - 1.0f);
    int lo = 0, hi = kBins - 1, found = 0, b_idx = 0;
    for (int it = 0; it < 5; ++it) {
      const int mid = (int)((float)(lo + hi) * 0.5f);
      float fL = 0.f, fU = 0.f;
      for (int j = 0; j < kBins; ++j) {
        const int off = j - mid;
        if (off < 0) continue;
        float cnt = (float)hist[j];
        if (j == kBins - 1) cnt -= 1.0f;
        const float zL = (float)off / kBins;
        const float zU = ((float)off + 1.0f) / kBins;
        if (zL > 0.f) fL += cnt * exp2f(log2f(zL) * p);
        fU += cnt * exp2f(log2f(zU) * p);
      }
      fL -= 1.0f;
      fU -= 1.0f;
      const bool go_right = fL > 0.f, go_left = fU < 0.f;
      const bool bracket = !go_right && !go_left;
      if (found == 0) {
        if (bracket) {
          b_idx = mid;
          found = 1;
        }
        if (go_right) lo = mid + 1;
        if (go_left) hi = mid - 1;
      }
    }
    const int b_sel = found ? b_idx : min(lo, kBins - 1);
    t_lo = t0 + (float)b_sel / kBins;
    t_hi = t0 + (float)min(b_sel + 1, kBins) / kBins;
  }
  t = 0.5f * (t_lo + t_hi);
}

// kernels/adadecode.py:12-35
__device__ __forceinline__ void halley_bisect(float& t, float& t_lo, float& t_hi, float a0,
                                              float a1, float a2, float c0, float c1) {
  const float ff = a0 - 1.0f;
  const float df = -c0 * a1;
  const float ddf = c0 * c1 * a2;
  if (ff > 0.f) t_lo = t;
  if (ff < 0.f) t_hi = t;
  const float new_t = t - (2.f * ff * df) / (2.f * df * df - ff * ddf);
  const bool good = (new_t > t_lo - 1e-6f) && (new_t < t_hi + 1e-6f);
  t = good ? new_t : 0.5f * (t_lo + t_hi);
}

// kernels/adadecode_paged_gaussian_tau.py:12-53
__device__ __forceinline__ float halley_unbounded(float t, float a0, float a1, float a2, float c0,
                                                  float c1) {
  const float ff = a0 - 1.0f;
  const float df = -c0 * a1;
  const float ddf = c0 * c1 * a2;
  const float hden = 2.0f * df * df - ff * ddf;
  float tn;
  if (fabsf(hden) > 1e-12f) tn = t - (2.0f * ff * df) / hden;
  else if (fabsf(df) > 1e-12f) tn = t - ff / df;
  else tn = t;
  if (!(tn == tn && fabsf(tn) < 1e20f)) tn = t;
  return tn;
}

__device__ void solve_tau_wave(const DecodeArgs& a, const float* __restrict__ sc, int n,
                               float tau_in, int* hist, float& tau_out) {
  const int lane = threadIdx.x & 63;
  const float alpha = a.alpha;
  const float c0 = 1.0f / (alpha - 1.0f);
  const float c1 = c0 - 1.0f;
  float t;
  if (a.tau_mode == 0) {
    float m = -1.0e6f;
    for (int c = lane; c < n; c += 64) m = fmaxf(m, sc[c]);
    const float gmax = wave_max(m);
    const float t0 = gmax - 1.0f;
    if (lane < kBins) hist[lane] = 0;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    for (int c = lane; c < n; c += 64) {
      const float f = (sc[c] - t0) * (float)kBins;
      if (f > -1.0f) atomicAdd(&hist[min((int)f, kBins - 1)], 1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
    __builtin_amdgcn_wave_barrier();
    float t_lo, t_hi;
    histogram_init(hist, gmax, alpha, t, t_lo, t_hi);
    for (int it = 0; it < a.iters; ++it) {
      float a0, a1, a2;
      accumulate(sc, n, t, alpha, c0, a0, a1, a2);
      halley_bisect(t, t_lo, t_hi, a0, a1, a2, c0, c1);
    }
  } else {
    t = tau_in;
    for (int it = 0; it < a.iters; ++it) {
      float a0, a1, a2;
      accumulate(sc, n, t, alpha, c0, a0, a1, a2);
      t = halley_unbounded(t, a0, a1, a2, c0, c1);
    }
  }
  tau_out = t;
}

// ---------------------------------------------------------------------------
// kernel 1: scores + tau
// ---------------------------------------------------------------------------

template <typename T, int LPR, int G>
__global__ __launch_bounds__(kThreads) void score_tau_kernel(DecodeArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SEGS = kThreads / LPR;
  constexpr int ROWS = SEGS * kUnroll;
  __shared__ int hist[kThreads / 64][kBins];
  const int seg = threadIdx.x / LPR;
  const int sl = threadIdx.x % LPR;
  const int col = sl * VEC;
  const int split = blockIdx.x;
  const int bkv = blockIdx.y;
  const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
  const int h0 = kvh * G;
  const int n = token_count(a, b, kvh);
  const int per = (n + a.splits - 1) / a.splits;
  const int c_start = split * per;
  const int c_end = min(c_start + per, n);

  if (c_start < c_end) {
    const T* qb = (const T*)a.q + b * a.qsb;
    float qv[G][VEC];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      Vec<T> x;
      x.load(qb + (h0 + g) * a.qsh + col);
#pragma unroll
      for (int i = 0; i < VEC; ++i) qv[g][i] = to_f<T>(from_f<T>(x.v[i] * a.qscale));
    }
    float slope[G];
    int q_idx = 0;
    if (a.slopes) {
      q_idx = (a.q_seqlens ? a.q_seqlens[b] : a.cache_seqlens[b * a.csb + kvh * a.csh]) - 1;
#pragma unroll
      for (int g = 0; g < G; ++g) slope[g] = a.slopes[h0 + g] * (a.alpha - 1.0f);
    }
    const int32_t* pi = a.page_indices + b * a.pisb + kvh * a.pish;
    const T* kh = (const T*)a.k + b * a.ksb + kvh * a.ksh;
    float* sc0 = a.ws_scores + ((int64_t)b * a.H + h0) * a.max_tokens;

    for (int c0 = c_start; c0 < c_end; c0 += ROWS) {
      VecRaw<T> kv[kUnroll];
      int64_t rows[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int c = c0 + u * SEGS + seg;
        rows[u] = (c < c_end) ? token_row(pi, c, a.page_size, a.row_limit) : -1;
        if (rows[u] >= 0) kv[u].load(kh + rows[u] * a.ksr + col);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int c = c0 + u * SEGS + seg;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float acc = 0.f;
          if (rows[u] >= 0) {
#pragma unroll
            for (int i = 0; i < VEC; ++i) acc += qv[g][i] * kv[u].get(i);
          }
          acc = seg_sum<LPR>(acc);
          if (c < c_end && sl == 0) {
            float s = acc;
            if (rows[u] < 0) s = -INFINITY;
            else if (a.slopes) s += slope[g] * (float)(rows[u] - q_idx);
            sc0[(int64_t)g * a.max_tokens + c] = s;
          }
        }
      }
    }
  }

  if (!last_arrival(&a.counters[bkv], a.splits)) return;

  // tau for the group's heads: one wave per head
  const int wid = threadIdx.x >> 6;
  for (int g0 = 0; g0 < G; g0 += kThreads / 64) {
    const int g = g0 + wid;
    if (g < G) {
      const int h = h0 + g;
      const float* sc = a.ws_scores + ((int64_t)b * a.H + h) * a.max_tokens;
      float* tp = a.tau + b * a.H + h;
      const float tin = (a.tau_mode == 1) ? *tp : 0.f;
      float tout;
      solve_tau_wave(a, sc, n, tin, hist[wid], tout);
      if ((threadIdx.x & 63) == 0) *tp = tout;
    }
  }
}

// ---------------------------------------------------------------------------
// kernel 2: support gather of V + deterministic split reduction
// ---------------------------------------------------------------------------

template <typename T, int LPR, int G>
__global__ __launch_bounds__(kThreads) void weighted_sum_kernel(DecodeArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SEGS = kThreads / LPR;
  constexpr int D = LPR * VEC;
  __shared__ int64_t sup_row[kThreads];
  __shared__ float sup_p[G][kThreads];
  __shared__ float red[SEGS][D];
  __shared__ int scan_scratch[kThreads / 64 + 1];

  const int tid = threadIdx.x;
  const int seg = tid / LPR;
  const int col = (tid % LPR) * VEC;
  const int split = blockIdx.x;
  const int bkv = blockIdx.y;
  const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
  const int h0 = kvh * G;
  const int n = token_count(a, b, kvh);
  const int per = (n + a.splits - 1) / a.splits;
  const int c_start = split * per;
  const int c_end = min(c_start + per, n);
  const float alpha = a.alpha;
  const float c0 = 1.0f / (alpha - 1.0f);

  float tau[G];
#pragma unroll
  for (int g = 0; g < G; ++g) tau[g] = a.tau[b * a.H + h0 + g];

  float acc[G][VEC];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[g][i] = 0.f;

  const int32_t* pi = a.page_indices + b * a.pisb + kvh * a.pish;
  const T* vh = (const T*)a.v + b * a.ksb + kvh * a.ksh;
  const float* sc0 = a.ws_scores + ((int64_t)b * a.H + h0) * a.max_tokens;
  int support = 0;

  for (int t0 = c_start; t0 < c_end; t0 += kThreads) {
    const int c = t0 + tid;
    float p[G];
    bool any = false;
    int64_t row = -1;
    if (c < c_end) {
      row = token_row(pi, c, a.page_size, a.row_limit);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float s = sc0[(int64_t)g * a.max_tokens + c];
        p[g] = 0.f;
        if (s > tau[g]) {
          p[g] = entmax_weight(s - tau[g], alpha, c0);
          any = true;
        }
      }
      if (row < 0) any = false;
    }
    int nsup;
    const int slot = block_excl_scan(any ? 1 : 0, scan_scratch, &nsup);
    if (any) {
      sup_row[slot] = row;
#pragma unroll
      for (int g = 0; g < G; ++g) sup_p[g][slot] = p[g];
    }
    __syncthreads();
    for (int j = seg; j < nsup; j += SEGS) {
      Vec<T> x;
      x.load(vh + sup_row[j] * a.ksr + col);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float w = sup_p[g][j];
#pragma unroll
        for (int i = 0; i < VEC; ++i) acc[g][i] += w * x.v[i];
      }
    }
    support += nsup;
    __syncthreads();
  }

  float* part = a.ws_partial + (((int64_t)b * a.H + h0) * a.splits + split) * D;
  if (support > 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) red[seg][col + i] = acc[g][i];
      __syncthreads();
      for (int e = tid; e < D; e += kThreads) {
        float r = 0.f;
        for (int s2 = 0; s2 < SEGS; ++s2) r += red[s2][e];
        part[(int64_t)g * a.splits * D + e] = r;
      }
      __syncthreads();
    }
  }
  if (tid == 0) a.ws_flags[(int64_t)bkv * a.splits + split] = support > 0 ? 1 : 0;

  if (!last_arrival(&a.counters[gridDim.y + bkv], a.splits)) return;

  const int* flags = a.ws_flags + (int64_t)bkv * a.splits;
  for (int e = tid; e < G * D; e += kThreads) {
    const int g = e / D, d = e % D;
    const float* pg = a.ws_partial + (((int64_t)b * a.H + h0 + g) * a.splits) * D + d;
    float r = 0.f;
    for (int s2 = 0; s2 < a.splits; ++s2)
      if (flags[s2]) r += pg[(int64_t)s2 * D];
    T* o = (T*)a.out + b * a.osb + (h0 + g) * a.osh;
    o[d] = from_f<T>(r);
  }
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

extern "C" int64_t ekv_decode_workspace_bytes(int B, int H, int Hkv, int D, int splits,
                                              int max_tokens) {
  const int64_t scores = (int64_t)B * H * max_tokens * 4;
  const int64_t partial = (int64_t)B * H * splits * D * 4;
  const int64_t flags = (int64_t)B * Hkv * splits * 4;
  const int64_t counters = (int64_t)2 * B * Hkv * 4;
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  return up(counters) + up(flags) + up(scores) + up(partial);
}

extern "C" int ekv_paged_entmax_decode(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k, const void* v,
    int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_row, int64_t kv_rows,
    const int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h, int n_slots,
    const int32_t* cache_seqlens, int64_t cs_stride_b, int64_t cs_stride_h,
    const int32_t* q_seqlens, const float* alibi_slopes, float* tau, int tau_mode, int iters,
    void* out, int64_t out_stride_b, int64_t out_stride_h, float alpha, float qscale,
    int page_size, int B, int H, int Hkv, int D, int splits, int max_tokens, void* workspace,
    int64_t workspace_bytes, int dtype, void* stream) {
  EKV_REQUIRE(q && k && v && page_indices && cache_seqlens && tau && out && workspace,
              "ekv_paged_entmax_decode: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "ekv_paged_entmax_decode: bad heads");
  EKV_REQUIRE(page_size > 0 && n_slots > 0 && splits > 0 && max_tokens > 0,
              "ekv_paged_entmax_decode: bad sizes");
  EKV_REQUIRE(tau_mode == 0 || tau_mode == 1, "ekv_paged_entmax_decode: tau_mode %d", tau_mode);
  EKV_REQUIRE(iters >= 0, "ekv_paged_entmax_decode: iters %d", iters);
  EKV_REQUIRE(alpha > 1.0f, "ekv_paged_entmax_decode: alpha must be > 1");
  EKV_REQUIRE(workspace_bytes >= ekv_decode_workspace_bytes(B, H, Hkv, D, splits, max_tokens),
              "ekv_paged_entmax_decode: workspace too small");
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  char* w = (char*)workspace;
  DecodeArgs a;
  a.counters = (int*)w;
  w += up((int64_t)2 * B * Hkv * 4);
  a.ws_flags = (int*)w;
  w += up((int64_t)B * Hkv * splits * 4);
  a.ws_scores = (float*)w;
  w += up((int64_t)B * H * max_tokens * 4);
  a.ws_partial = (float*)w;
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
  hipStream_t s = (hipStream_t)stream;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    return dispatch_lpr<T>(D, [&](auto lpr) {
      constexpr int LPR = decltype(lpr)::value;
      return dispatch_group(H / Hkv, [&](auto gv) {
        constexpr int G = decltype(gv)::value;
        dim3 grid(splits, B * Hkv);
        hipLaunchKernelGGL((score_tau_kernel<T, LPR, G>), grid, dim3(kThreads), 0, s, a);
        int rc = check_launch("score_tau_kernel");
        if (rc) return rc;
        hipLaunchKernelGGL((weighted_sum_kernel<T, LPR, G>), grid, dim3(kThreads), 0, s, a);
        return check_launch("weighted_sum_kernel");
      });
    });
  });
}
