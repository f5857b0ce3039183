// Row-wise alpha-entmax forward and backward (dense utilities).
//
// Forward (kernels/triton_entmax.py:364-533): for each row x of length n,
// z = (alpha - 1) x and y = [z - tau]_+^(1/(alpha-1)) with tau such that
// sum(y) = 1.  The reference runs n_iter (default 2) hybrid Halley/secant
// steps from a histogram initialisation, so its output approaches exact
// entmax; this kernel solves tau exactly:
//   * alpha = 2 and alpha = 1.5: support refinement from below.  tau* >= max - 1
//     (the top element alone contributes 1), so start at t = max - 1.  Each
//     pass sums d = z - t over S = {z > t} (count, sum d, sum d^2, min d) and
//     takes the closed-form root t + delta of sum_S (z - t')^(1/(alpha-1)) = 1;
//     when t + delta lies below every element of S it is tau* exactly (the
//     sort-based solution, Peters et al. 2019, Alg. 2, without the sort).
//     Otherwise S is too large and t moves to a point that stays <= tau*:
//     the sparsemax root of S (Michelot's step) or, for 1.5-entmax, a Newton
//     step on the convex, decreasing f(t) = sum [z - t]_+^2 - 1;
//   * other alpha: safeguarded Halley on f(t) = sum [z - t]_+^(1/(alpha-1)) - 1
//     over [max - 1, max - n^(1-alpha)] to fp32 resolution.
// Backward (kernels/triton_entmax.py:536-612): u = y^(2 - alpha) on the
// support (1 for alpha = 2, sqrt(y) for 1.5), dx = u dy - (sum u dy / sum u) u.
//
// One workgroup of 256 threads per row; the row's z stays in LDS when it fits
// (kRowCache floats), otherwise it is recomputed from x on every pass.
#include "ekv_common.h"
#include "../../include/entmaxkv.h"

using namespace ekv;

namespace {

constexpr int kThreads = 256;
constexpr int kRowCache = 16384;  // floats of z cached in LDS (64 KB)
constexpr int kMaxRounds = 64;

template <typename T>
struct Row {
  const T* x;
  const float* zc;  // LDS copy or null
  float am1;
  __device__ __forceinline__ float z(int i) const { return zc ? zc[i] : to_f<T>(x[i]) * am1; }
};

__device__ __forceinline__ float block_max_f(float v, float* scratch) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_max(v);
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  float r = scratch[0];
  for (int w = 1; w < kThreads / 64; ++w) r = fmaxf(r, scratch[w]);
  __syncthreads();
  return r;
}

// Sums over S = {z > t} of 1, d, d^2 with d = z - t, and min_S d (fixed-order
// block reductions).
template <typename T>
__device__ __forceinline__ void support_sums(const Row<T>& r, int n, float t, float* scratch,
                                             float& k, float& s1, float& s2, float& dmin) {
  float a = 0.f, b = 0.f, c = 0.f, m = INFINITY;
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const float d = r.z(i) - t;
    if (d > 0.f) {
      a += 1.f;
      b += d;
      c += d * d;
      m = fminf(m, d);
    }
  }
  k = block_sum(a, scratch);
  s1 = block_sum(b, scratch);
  s2 = block_sum(c, scratch);
  dmin = -block_max_f(-m, scratch);
}

// f and its first two derivatives for the generic alpha: sums over {z > t} of
// d^c, d^(c-1), d^(c-2) with d = z - t, c = 1 / (alpha - 1).
template <typename T>
__device__ __forceinline__ void generic_sums(const Row<T>& r, int n, float t, float c,
                                             float* scratch, float& a0, float& a1, float& a2) {
  float x0 = 0.f, x1 = 0.f, x2 = 0.f;
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const float d = r.z(i) - t;
    if (d > 0.f) {
      const float l = log2f(d);
      x0 += exp2f(l * c);
      x1 += exp2f(l * (c - 1.f));
      x2 += exp2f(l * (c - 2.f));
    }
  }
  a0 = block_sum(x0, scratch);
  a1 = block_sum(x1, scratch);
  a2 = block_sum(x2, scratch);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void entmax_fwd_kernel(const T* __restrict__ x,
                                                              T* __restrict__ y, int64_t sx,
                                                              int64_t sy, int n, float alpha,
                                                              float* __restrict__ tau_out) {
  extern __shared__ float zc[];
  __shared__ float scratch[16];
  const int64_t row = blockIdx.x;
  const bool cached = n <= kRowCache;
  Row<T> r{x + row * sx, cached ? zc : nullptr, alpha - 1.0f};
  float m = -INFINITY;
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const float z = to_f<T>(r.x[i]) * r.am1;
    if (cached) zc[i] = z;
    m = fmaxf(m, z);
  }
  m = block_max_f(m, scratch);  // also orders the LDS writes before the reads
  float t;
  if (alpha == 2.0f || alpha == 1.5f) {
    t = m - 1.0f;
    for (int round = 0; round < kMaxRounds; ++round) {
      float k, s1, s2, dmin;
      support_sums(r, n, t, scratch, k, s1, s2, dmin);
      float delta, step;
      if (alpha == 2.0f) {
        delta = (s1 - 1.0f) / k;
        step = delta;
      } else {
        // k e^2 - 2 s1 e + (s2 - 1) = 0, smaller root in rationalised form
        const float c0 = s2 - 1.0f;
        const float disc = s1 * s1 - k * c0;
        delta = disc >= 0.f ? c0 / (s1 + sqrtf(disc)) : INFINITY;
        step = c0 / (2.0f * s1);  // Newton
      }
      if (delta < dmin) {  // the root keeps all of S: exact
        t += delta;
        break;
      }
      const float nt = t + step;
      if (!(nt > t)) break;  // fp32 stall
      t = nt;
    }
  } else {
    // bracket [max - 1, max - n^(1 - alpha)]: f(max - n^(1-alpha)) <= n * n^-1 = 1.
    // Halley steps that leave the bracket, or fail to halve it over two
    // steps, are replaced by a bisection, geometric in the gap max - t while
    // the gap spans more than a factor 4 (roots close to the maximum).
    const float c = 1.0f / (alpha - 1.0f);
    float lo = m - 1.0f;
    float hi = m - exp2f((1.0f - alpha) * log2f((float)n));
    if (!(hi > lo)) hi = m;
    float w1 = hi - lo, w2 = w1;
    t = lo;
    for (int it = 0; it < kMaxRounds; ++it) {
      float a0, a1, a2;
      generic_sums(r, n, t, c, scratch, a0, a1, a2);
      const float f = a0 - 1.0f;
      if (f > 0.f) lo = fmaxf(lo, t);
      else hi = fminf(hi, t);
      const float w = hi - lo;
      const float scale = fmaxf(1.0f, fabsf(t));
      if (w <= 2.4e-7f * scale) {
        t = 0.5f * (lo + hi);
        break;
      }
      const float df = -c * a1, ddf = c * (c - 1.0f) * a2;
      const float den = 2.0f * df * df - f * ddf;
      float cand = den != 0.f ? t - 2.0f * f * df / den : lo;
      if (!(cand > lo && cand < hi) || w > 0.5f * w2) {
        const float glo = m - hi, ghi = m - lo;
        cand = (glo > 0.f && ghi > 4.0f * glo) ? m - sqrtf(glo * ghi) : 0.5f * (lo + hi);
      }
      if (fabsf(cand - t) <= 1.2e-7f * scale) {
        t = cand;
        break;
      }
      w2 = w1;
      w1 = w;
      t = cand;
    }
  }
  if (tau_out && threadIdx.x == 0) tau_out[row] = t;
  T* yr = y + row * sy;
  const float c = 1.0f / (alpha - 1.0f);
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const float d = r.z(i) - t;
    float v = 0.f;
    if (d > 0.f) {
      if (alpha == 2.0f) v = d;
      else if (alpha == 1.5f) v = d * d;
      else v = exp2f(log2f(d) * c);
    }
    yr[i] = from_f<T>(v);
  }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void entmax_bwd_kernel(const T* __restrict__ y,
                                                              const T* __restrict__ dy,
                                                              T* __restrict__ dx, int64_t sy,
                                                              int64_t sdy, int64_t sdx, int n,
                                                              float alpha) {
  __shared__ float scratch[16];
  const int64_t row = blockIdx.x;
  const T* yr = y + row * sy;
  const T* gr = dy + row * sdy;
  auto weight = [&](float yv) -> float {
    if (!(yv > 0.f)) return 0.f;
    if (alpha == 2.0f) return 1.f;
    if (alpha == 1.5f) return sqrtf(yv);
    return exp2f(log2f(yv) * (2.0f - alpha));
  };
  float s_ug = 0.f, s_u = 0.f;
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const float u = weight(to_f<T>(yr[i]));
    s_ug += u * to_f<T>(gr[i]);
    s_u += u;
  }
  s_ug = block_sum(s_ug, scratch);
  s_u = block_sum(s_u, scratch);
  const float scalar = s_ug / s_u;
  T* xr = dx + row * sdx;
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const float u = weight(to_f<T>(yr[i]));
    xr[i] = from_f<T>(u * to_f<T>(gr[i]) - scalar * u);
  }
}

}  // namespace

extern "C" int ekv_entmax_rows_forward(const void* x, int64_t x_row_stride, void* y,
                                       int64_t y_row_stride, int64_t rows, int n, float alpha,
                                       float* tau_out, int dtype, void* stream) {
  EKV_REQUIRE(x && y, "ekv_entmax_rows_forward: null pointer");
  EKV_REQUIRE(rows >= 0 && n > 0, "ekv_entmax_rows_forward: bad sizes (%lld rows of %d)",
              (long long)rows, n);
  EKV_REQUIRE(alpha > 1.0f, "ekv_entmax_rows_forward: alpha must be > 1");
  EKV_REQUIRE(rows <= 0x7fffffff, "ekv_entmax_rows_forward: too many rows");
  if (rows == 0) return EKV_OK;
  hipStream_t s = (hipStream_t)stream;
  const size_t lds = n <= kRowCache ? (size_t)n * sizeof(float) : 0;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    hipLaunchKernelGGL((entmax_fwd_kernel<T>), dim3((unsigned)rows), dim3(kThreads), lds, s,
                       (const T*)x, (T*)y, x_row_stride, y_row_stride, n, alpha, tau_out);
    return check_launch("entmax_fwd_kernel");
  });
}

extern "C" int ekv_entmax_rows_backward(const void* y, int64_t y_row_stride, const void* dy,
                                        int64_t dy_row_stride, void* dx, int64_t dx_row_stride,
                                        int64_t rows, int n, float alpha, int dtype,
                                        void* stream) {
  EKV_REQUIRE(y && dy && dx, "ekv_entmax_rows_backward: null pointer");
  EKV_REQUIRE(rows >= 0 && n > 0 && rows <= 0x7fffffff, "ekv_entmax_rows_backward: bad sizes");
  EKV_REQUIRE(alpha > 1.0f, "ekv_entmax_rows_backward: alpha must be > 1");
  if (rows == 0) return EKV_OK;
  hipStream_t s = (hipStream_t)stream;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    hipLaunchKernelGGL((entmax_bwd_kernel<T>), dim3((unsigned)rows), dim3(kThreads), 0, s,
                       (const T*)y, (const T*)dy, (T*)dx, y_row_stride, dy_row_stride,
                       dx_row_stride, n, alpha);
    return check_launch("entmax_bwd_kernel");
  });
}
