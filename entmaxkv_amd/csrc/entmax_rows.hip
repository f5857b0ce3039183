// Row-wise alpha-entmax forward and backward (dense utilities).
//
// Forward (kernels/triton_entmax.py:364-533): for each row x of length n,
// z = (alpha - 1) x and y = [z - tau]_+^(1/(alpha-1)) with tau such that
// sum(y) = 1.  The reference runs n_iter (default 2) hybrid Halley/secant
// steps from a histogram initialisation, so its output approaches exact
// entmax; this kernel solves tau exactly:
//   * alpha = 2 and alpha = 1.5: support refinement from below.  tau* >= max - 1
//     (the top element alone contributes 1); a 16-bin histogram of the values
//     in (max - 1, max] gives a closer start that is still <= tau*.  Each
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
// Workgroups of 256 threads, one row at a time.  Rows of up to 8192 elements
// stay in registers (the next power of two of n / 256 per thread); longer
// rows keep z in LDS when it fits (kRowCache floats), otherwise recompute it
// from x on every pass.  Each pass ends in one block reduction of four values
// (one barrier).  The forward of register rows read in 16-byte chunks runs
// persistent workgroups that load their next row during the current one.
#include "ekv_common.h"

#include <initializer_list>
#include <utility>
#include "../../include/entmaxkv.h"

using namespace ekv;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRowCache = 16384;  // floats of z cached in LDS (64 KB)
constexpr int kMaxRounds = 64;
constexpr int kMaxRegVals = 32;   // values per thread kept in registers (n <= 8192)

// Block-wide reduction of (sum, sum, sum, min) with one barrier: each wave
// reduces in registers and writes one float4; the buffers alternate, so a
// buffer is rewritten only after every thread has passed the next barrier.
struct Reducer {
  float4 (*buf)[kWaves];  // [2][kWaves] in LDS
  int parity = 0;
  __device__ __forceinline__ float4 sum3_min(float a, float b, float c, float d) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    a = wave_sum(a);
    b = wave_sum(b);
    c = wave_sum(c);
    d = -wave_max(-d);
    if (lane == 0) buf[parity][wid] = make_float4(a, b, c, d);
    __syncthreads();
    float4 r = buf[parity][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      const float4 o = buf[parity][w];
      r.x += o.x;
      r.y += o.y;
      r.z += o.z;
      r.w = fminf(r.w, o.w);
    }
    parity ^= 1;
    return r;
  }
};

// Element of value j (chunk j / E, lane j % E) of this thread: chunks of E
// contiguous elements, chunk c of thread t at (c * kThreads + t) * E.
template <int E>
__device__ __forceinline__ int elem_index(int j) {
  return ((j / E) * kThreads + (int)threadIdx.x) * E + j % E;
}

// Loads VPT values of a row into registers, chunks of E elements (E > 1:
// 16-byte loads, n % E == 0 and 16-byte aligned rows).  Every load is issued
// unconditionally (out-of-range chunks re-read the last one), so all of them
// are in flight together; out-of-range values become `fill`.
template <typename T, int VPT, int E>
__device__ __forceinline__ void load_row(const T* __restrict__ p, int n, float scale, float fill,
                                         float (&v)[VPT]) {
#pragma unroll
  for (int c = 0; c < VPT / E; ++c) {
    const int i0 = (c * kThreads + (int)threadIdx.x) * E;
    const int ic = min(i0, n - E);
    if constexpr (E > 1) {
      Vec<T> t;
      t.load(p + ic);
#pragma unroll
      for (int e = 0; e < E; ++e) v[c * E + e] = i0 < n ? t.v[e] * scale : fill;
    } else {
      const float t = to_f<T>(p[ic]) * scale;
      v[c] = i0 < n ? t : fill;
    }
  }
}

// Stores f(j) for the in-range values j of this thread.
template <typename T, int VPT, int E, typename F>
__device__ __forceinline__ void store_row(T* __restrict__ p, int n, F f) {
#pragma unroll
  for (int c = 0; c < VPT / E; ++c) {
    const int i0 = (c * kThreads + (int)threadIdx.x) * E;
    if (i0 >= n) continue;
    if constexpr (E > 1) {
      Vec<T> t;
#pragma unroll
      for (int e = 0; e < E; ++e) t.v[e] = f(c * E + e);
      t.store(p + i0);
    } else {
      p[i0] = from_f<T>(f(c));
    }
  }
}

// The row's z = (alpha - 1) x held in registers (see elem_index).  Slots
// past the row's end hold -inf, which every pass skips (z - t > 0 fails), so
// each() visits all slots without a range check.
template <int VPT, int E>
struct RegVals {
  float v[VPT];
  int n;
  template <typename F> __device__ __forceinline__ void each(F f) const {
#pragma unroll
    for (int j = 0; j < VPT; ++j) f(elem_index<E>(j), v[j]);
  }
};

// The row's z read from LDS (zc non-null) or recomputed from x.
template <typename T>
struct MemVals {
  const T* x;
  const float* zc;
  float am1;
  int n;
  template <typename F> __device__ __forceinline__ void each(F f) const {
    for (int i = threadIdx.x; i < n; i += kThreads) f(i, zc ? zc[i] : to_f<T>(x[i]) * am1);
  }
};

constexpr int kStartBins = 16;

// A start t <= tau* for alpha 2 / 1.5 closer than max - 1: the values in
// (m - 1, m] are counted in kStartBins bins of width 1/kStartBins (`hbin`,
// zero and visible on entry), and f is bounded from below at each bin edge
// e_b by counting every value at its bin's lower edge (the maximum itself at
// m); the largest edge whose bound exceeds 1 (with a 1e-3 margin for the
// fp32 binning) is <= tau*, since f decreases.
template <typename V>
__device__ __forceinline__ float start_tau(const V& vals, float m, float alpha, unsigned* hbin) {
  const float t0 = m - 1.0f;
  vals.each([&](int, float z) {
    const float d = z - t0;
    if (d > 0.f) atomicAdd(&hbin[min(kStartBins - 1, (int)(d * kStartBins))], 1u);
  });
  __syncthreads();
  unsigned cnt[kStartBins];
#pragma unroll
  for (int j = 0; j < kStartBins; ++j) cnt[j] = hbin[j];
  cnt[kStartBins - 1] -= 1;  // the maximum lies in the top bin; it is counted at m
  float t = t0;
#pragma unroll
  for (int b = 1; b < kStartBins; ++b) {
    const float e = t0 + (float)b / kStartBins;
    const float dm = m - e;
    float f = alpha == 2.0f ? dm : dm * dm;
#pragma unroll
    for (int j = b + 1; j < kStartBins; ++j) {
      const float w = (float)(j - b) / kStartBins;
      f += (float)cnt[j] * (alpha == 2.0f ? w : w * w);
    }
    if (f >= 1.001f) t = e;
  }
  return t;
}

// Exact tau of one row from its maximum m (see the file comment).
template <typename V>
__device__ __forceinline__ float solve_row_tau(const V& vals, int n, float m, float alpha,
                                               Reducer& red, unsigned* hbin) {
  float t;
  if (alpha == 2.0f || alpha == 1.5f) {
    t = start_tau(vals, m, alpha, hbin);
    for (int round = 0; round < kMaxRounds; ++round) {
      float a = 0.f, b = 0.f, c = 0.f, mn = INFINITY;
      vals.each([&](int, float z) {
        const float d = z - t;
        if (d > 0.f) {
          a += 1.f;
          b += d;
          c += d * d;
          mn = fminf(mn, d);
        }
      });
      const float4 r = red.sum3_min(a, b, c, mn);
      const float k = r.x, s1 = r.y, s2 = r.z, dmin = r.w;
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
    return t;
  }
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
    float x0 = 0.f, x1 = 0.f, x2 = 0.f;
    vals.each([&](int, float z) {
      const float d = z - t;
      if (d > 0.f) {
        const float l = log2f(d);
        x0 += exp2f(l * c);
        x1 += exp2f(l * (c - 1.f));
        x2 += exp2f(l * (c - 2.f));
      }
    });
    const float4 r = red.sum3_min(x0, x1, x2, 0.f);
    const float f = r.x - 1.0f;
    if (f > 0.f) lo = fmaxf(lo, t);
    else hi = fminf(hi, t);
    const float w = hi - lo;
    const float scale = fmaxf(1.0f, fabsf(t));
    if (w <= 2.4e-7f * scale) {
      t = 0.5f * (lo + hi);
      break;
    }
    const float df = -c * r.y, ddf = c * (c - 1.0f) * r.z;
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
  return t;
}

__device__ __forceinline__ float entmax_value(float d, float alpha) {
  if (!(d > 0.f)) return 0.f;
  if (alpha == 2.0f) return d;
  if (alpha == 1.5f) return d * d;
  return exp2f(log2f(d) * (1.0f / (alpha - 1.0f)));
}

// VPT > 0: the row (n <= VPT * kThreads) in registers, chunks of E; VPT ==
// 0: in LDS when it fits (kRowCache floats of dynamic LDS), else re-read from
// x every pass.
template <typename T, int VPT, int E>
__global__ __launch_bounds__(kThreads) void entmax_fwd_kernel(const T* __restrict__ x,
                                                              T* __restrict__ y, int64_t sx,
                                                              int64_t sy, int n, float alpha,
                                                              float* __restrict__ tau_out) {
  __shared__ float4 rbuf[2][kWaves];
  __shared__ unsigned hbin[kStartBins];
  Reducer red{rbuf};
  if (threadIdx.x < kStartBins) hbin[threadIdx.x] = 0u;  // visible after the max reduction
  const int64_t row = blockIdx.x;
  const T* xr = x + row * sx;
  T* yr = y + row * sy;
  const float am1 = alpha - 1.0f;
  float m = -INFINITY;
  float t;
  if constexpr (VPT > 0) {
    RegVals<VPT, E> vals;
    vals.n = n;
    load_row<T, VPT, E>(xr, n, am1, -INFINITY, vals.v);
#pragma unroll
    for (int j = 0; j < VPT; ++j) m = fmaxf(m, vals.v[j]);
    m = -red.sum3_min(0.f, 0.f, 0.f, -m).w;
    t = solve_row_tau(vals, n, m, alpha, red, hbin);
    store_row<T, VPT, E>(yr, n, [&](int j) { return entmax_value(vals.v[j] - t, alpha); });
  } else {
    extern __shared__ float zc[];
    const bool cached = n <= kRowCache;
    for (int i = threadIdx.x; i < n; i += kThreads) {
      const float z = to_f<T>(xr[i]) * am1;
      if (cached) zc[i] = z;
      m = fmaxf(m, z);
    }
    m = -red.sum3_min(0.f, 0.f, 0.f, -m).w;  // its barrier orders the LDS writes
    MemVals<T> vals{xr, cached ? zc : nullptr, am1, n};
    t = solve_row_tau(vals, n, m, alpha, red, hbin);
    vals.each([&](int i, float z) { yr[i] = from_f<T>(entmax_value(z - t, alpha)); });
  }
  if (tau_out && threadIdx.x == 0) tau_out[row] = t;
}

// Rows held in registers with 16-byte chunks, several rows per workgroup
// (row blockIdx.x, then every gridDim.x-th): the next row's raw chunks are
// loaded while the current row's tau is solved, so each CU keeps reading
// while its workgroups sit in the reductions.  The grid holds as many
// workgroups as fit on the device at once.
template <typename T, int VPT, int E>
__global__ __launch_bounds__(kThreads) void entmax_fwd_pipe_kernel(
    const T* __restrict__ x, T* __restrict__ y, int64_t sx, int64_t sy, int n, float alpha,
    float* __restrict__ tau_out, int rows) {
  static_assert(E > 1 && VPT % E == 0, "16-byte chunks only");
  constexpr int C = VPT / E;
  __shared__ float4 rbuf[2][kWaves];
  __shared__ unsigned hbin[2][kStartBins];
  Reducer red{rbuf};
  const float am1 = alpha - 1.0f;
  VecRaw<T> nxt[C];
  auto fetch = [&](int r) {
    const T* xr = x + (int64_t)r * sx;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int i0 = (c * kThreads + (int)threadIdx.x) * E;
      nxt[c].load(xr + min(i0, n - E));
    }
  };
  int row = blockIdx.x;
  if (row < rows) fetch(row);
  for (int it = 0; row < rows; row += gridDim.x, ++it) {
    // hbin[it & 1] was last read two rows ago, before at least one barrier
    if (threadIdx.x < kStartBins) hbin[it & 1][threadIdx.x] = 0u;
    RegVals<VPT, E> vals;
    vals.n = n;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const int i0 = (c * kThreads + (int)threadIdx.x) * E;
#pragma unroll
      for (int e = 0; e < E; ++e) vals.v[c * E + e] = i0 < n ? nxt[c].get(e) * am1 : -INFINITY;
    }
    if (row + (int)gridDim.x < rows) fetch(row + gridDim.x);
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPT; ++j) m = fmaxf(m, vals.v[j]);
    m = -red.sum3_min(0.f, 0.f, 0.f, -m).w;  // its barrier publishes the zeroed bins
    const float t = solve_row_tau(vals, n, m, alpha, red, hbin[it & 1]);
    store_row<T, VPT, E>(y + (int64_t)row * sy, n,
                         [&](int j) { return entmax_value(vals.v[j] - t, alpha); });
    if (tau_out && threadIdx.x == 0) tau_out[row] = t;
  }
}

__device__ __forceinline__ float entmax_grad_weight(float yv, float alpha) {
  if (!(yv > 0.f)) return 0.f;
  if (alpha == 2.0f) return 1.f;
  if (alpha == 1.5f) return sqrtf(yv);
  return exp2f(log2f(yv) * (2.0f - alpha));
}

// VPT > 0: y and dy read once into registers (n <= VPT * kThreads, chunks of
// E); VPT == 0: two passes over global memory.
template <typename T, int VPT, int E>
__global__ __launch_bounds__(kThreads) void entmax_bwd_kernel(const T* __restrict__ y,
                                                              const T* __restrict__ dy,
                                                              T* __restrict__ dx, int64_t sy,
                                                              int64_t sdy, int64_t sdx, int n,
                                                              float alpha) {
  __shared__ float4 rbuf[2][kWaves];
  Reducer red{rbuf};
  const int64_t row = blockIdx.x;
  const T* yr = y + row * sy;
  const T* gr = dy + row * sdy;
  T* xr = dx + row * sdx;
  float s_ug = 0.f, s_u = 0.f;
  if constexpr (VPT > 0) {
    float u[VPT], g[VPT];
    load_row<T, VPT, E>(yr, n, 1.0f, 0.f, u);
    load_row<T, VPT, E>(gr, n, 1.0f, 0.f, g);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      u[j] = entmax_grad_weight(u[j], alpha);
      s_ug += u[j] * g[j];
      s_u += u[j];
    }
    const float4 r = red.sum3_min(s_ug, s_u, 0.f, 0.f);
    const float scalar = r.x / r.y;
    store_row<T, VPT, E>(xr, n, [&](int j) { return u[j] * g[j] - scalar * u[j]; });
  } else {
    for (int i = threadIdx.x; i < n; i += kThreads) {
      const float uv = entmax_grad_weight(to_f<T>(yr[i]), alpha);
      s_ug += uv * to_f<T>(gr[i]);
      s_u += uv;
    }
    const float4 r = red.sum3_min(s_ug, s_u, 0.f, 0.f);
    const float scalar = r.x / r.y;
    for (int i = threadIdx.x; i < n; i += kThreads) {
      const float uv = entmax_grad_weight(to_f<T>(yr[i]), alpha);
      xr[i] = from_f<T>(uv * to_f<T>(gr[i]) - scalar * uv);
    }
  }
}

// Workgroups of a persistent row kernel: as many as are resident on the
// device at once (occupancy per CU, queried once per kernel), at most `rows`.
template <typename K>
unsigned resident_grid(K kernel, int64_t rows) {
  static int per_cu = -1;  // one per kernel instantiation; every device gets the same figure
  if (per_cu < 0) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel, kThreads, 0) != hipSuccess)
      nb = 1;
    per_cu = nb < 1 ? 1 : nb;
  }
  const int64_t slots = (int64_t)per_cu * device_cus();
  return (unsigned)(rows < slots ? rows : slots);
}

// Registers per thread for a row of n: the next power of two of n / kThreads
// (at most kMaxRegVals), 0 for rows that do not fit.
int values_per_thread(int n) {
  if (n > kMaxRegVals * kThreads) return 0;
  int v = 1;
  while (v * kThreads < n) v *= 2;
  return v;
}

// 16-byte chunks when every row is aligned and n is a multiple of the chunk
// (and at least one chunk per thread fits VPT).
template <typename T>
bool rows_vectorisable(int n, int vpt, std::initializer_list<std::pair<const void*, int64_t>> rows) {
  constexpr int E = 16 / sizeof(T);
  if (vpt < E || n % E) return false;
  for (const auto& r : rows)
    if (((uintptr_t)r.first % 16) || ((r.second * (int64_t)sizeof(T)) % 16)) return false;
  return true;
}

template <typename F>
int dispatch_vpt(int vpt, F&& f) {
  switch (vpt) {
    case 1: return f(std::integral_constant<int, 1>{});
    case 2: return f(std::integral_constant<int, 2>{});
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    case 16: return f(std::integral_constant<int, 16>{});
    case 32: return f(std::integral_constant<int, 32>{});
    default: return f(std::integral_constant<int, 0>{});
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
  const int vpt = values_per_thread(n);
  const size_t lds = vpt == 0 && n <= kRowCache ? (size_t)n * sizeof(float) : 0;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    const bool vec = rows_vectorisable<T>(n, vpt, {{x, x_row_stride}, {y, y_row_stride}});
    return dispatch_vpt(vpt, [&](auto vv) {
      constexpr int VPT = decltype(vv)::value;
      constexpr int EV = 16 / sizeof(T);
      if constexpr (VPT >= EV) {
        if (vec) {
          const unsigned grid = resident_grid(entmax_fwd_pipe_kernel<T, VPT, EV>, rows);
          hipLaunchKernelGGL((entmax_fwd_pipe_kernel<T, VPT, EV>), dim3(grid), dim3(kThreads), 0,
                             s, (const T*)x, (T*)y, x_row_stride, y_row_stride, n, alpha,
                             tau_out, (int)rows);
          return check_launch("entmax_fwd_pipe_kernel");
        }
      }
      hipLaunchKernelGGL((entmax_fwd_kernel<T, VPT, 1>), dim3((unsigned)rows), dim3(kThreads),
                         lds, s, (const T*)x, (T*)y, x_row_stride, y_row_stride, n, alpha,
                         tau_out);
      return check_launch("entmax_fwd_kernel");
    });
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
  const int vpt = values_per_thread(n);
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    const bool vec = rows_vectorisable<T>(n, vpt, {{y, y_row_stride}, {dy, dy_row_stride},
                                                   {dx, dx_row_stride}});
    return dispatch_vpt(vpt, [&](auto vv) {
      constexpr int VPT = decltype(vv)::value;
      constexpr int EV = 16 / sizeof(T);
      if constexpr (VPT >= EV) {
        if (vec) {
          hipLaunchKernelGGL((entmax_bwd_kernel<T, VPT, EV>), dim3((unsigned)rows),
                             dim3(kThreads), 0, s, (const T*)y, (const T*)dy, (T*)dx,
                             y_row_stride, dy_row_stride, dx_row_stride, n, alpha);
          return check_launch("entmax_bwd_kernel");
        }
      }
      hipLaunchKernelGGL((entmax_bwd_kernel<T, VPT, 1>), dim3((unsigned)rows), dim3(kThreads), 0,
                         s, (const T*)y, (const T*)dy, (T*)dx, y_row_stride, dy_row_stride,
                         dx_row_stride, n, alpha);
      return check_launch("entmax_bwd_kernel");
    });
  });
}
