// Append of one K/V row with the recompute of its page's statistics, shared
// by the standalone append launch (page_stats.hip) and the fused top-k launch
// (decode_device.h).  Replaces the torch.cat + last-page recompute of
// PagedKVCache.append (kv_cache.py:72-116): min, max, mean and the population
// standard deviation (clamped to >= 1e-6) of the page's rows, accumulated in
// fp32 and rounded once to the key dtype.
#pragma once

#include "ekv_common.h"

namespace ekv {

// The [D] rows of one page in the four statistics tensors.
template <typename T>
struct PageStatRows {
  T* mn;
  T* mx;
  T* mean;
  T* sd;
};

// One row segment of LPR lanes (this lane covers elements col .. col + VEC):
// writes row `pos` of K and V, where kh + r * ksr (vh likewise) addresses
// the rows r of pos's page, and recomputes that page's statistics (the new
// row taken from registers).
template <typename T, int LPR>
__device__ __forceinline__ void append_row(const T* __restrict__ kn, const T* __restrict__ vn,
                                           T* kh, T* vh, int64_t ksr, int pos, int page_size,
                                           PageStatRows<T> st, int col) {
  constexpr int VEC = 16 / sizeof(T);
  Vec<T> kx;
  kx.load(kn + col);
  // raw 16-byte copies keep the stored bits identical to the inputs
  *reinterpret_cast<uint4*>(kh + (int64_t)pos * ksr + col) = *reinterpret_cast<const uint4*>(kn + col);
  *reinterpret_cast<uint4*>(vh + (int64_t)pos * ksr + col) = *reinterpret_cast<const uint4*>(vn + col);

  const int page = pos / page_size;
  const int r0 = page * page_size;
  const int n_rows = pos - r0 + 1;
  float mn[VEC], mx[VEC], sm[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    mn[i] = kx.v[i];
    mx[i] = kx.v[i];
    sm[i] = 0.f;
  }
  for (int r = r0; r < pos; ++r) {
    Vec<T> x;
    x.load(kh + (int64_t)r * ksr + col);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      mn[i] = fminf(mn[i], x.v[i]);
      mx[i] = fmaxf(mx[i], x.v[i]);
      sm[i] += x.v[i];
    }
  }
#pragma unroll
  for (int i = 0; i < VEC; ++i) sm[i] += kx.v[i];
  float mean[VEC], m2[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    mean[i] = sm[i] / (float)n_rows;
    m2[i] = 0.f;
  }
  for (int r = r0; r < pos; ++r) {
    Vec<T> x;
    x.load(kh + (int64_t)r * ksr + col);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float d = x.v[i] - mean[i];
      m2[i] += d * d;
    }
  }
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    float d = kx.v[i] - mean[i];
    m2[i] += d * d;
  }
  Vec<T> o;
#pragma unroll
  for (int i = 0; i < VEC; ++i) o.v[i] = mn[i];
  o.store(st.mn + col);
#pragma unroll
  for (int i = 0; i < VEC; ++i) o.v[i] = mx[i];
  o.store(st.mx + col);
#pragma unroll
  for (int i = 0; i < VEC; ++i) o.v[i] = mean[i];
  o.store(st.mean + col);
  const float inv_n = 1.0f / (float)n_rows;
#pragma unroll
  for (int i = 0; i < VEC; ++i) o.v[i] = fmaxf(sqrtf(m2[i] * inv_n), 1e-6f);
  o.store(st.sd + col);
}

}  // namespace ekv
