// Per-page key statistics: build over a page range, and in-place append.
//
// Replaces the Python page loop of PagedKVCache.initialize (kv_cache.py:58-70)
// and the torch.cat + last-page recompute of PagedKVCache.append
// (kv_cache.py:72-116).  For page p the statistics cover cache rows
// [p*ps, min((p+1)*ps, seq_len)): min, max, mean and the population standard
// deviation clamped to >= 1e-6, all accumulated in fp32 and rounded once to the
// key dtype.  With per-sequence lengths (seq_lens[b]) each batch element's
// pages end at its own length.
//
// HBM: each page's rows are read twice (min/max/sum, then the centred second
// moment); the second read hits L2 because a workgroup owns whole pages.
#include "ekv_common.h"
#include "append_device.h"
#include "../../include/entmaxkv.h"

using namespace ekv;

namespace {

struct StatsPtrs {
  void* kmin;
  void* kmax;
  void* kmean;
  void* kstd;
};

template <typename T, int LPR>
__device__ __forceinline__ void page_stats_one(const T* __restrict__ krow0, int64_t ksr, int n_rows,
                                               T* smin, T* smax, T* smean, T* sstd, int col) {
  constexpr int VEC = 16 / sizeof(T);
  float mn[VEC], mx[VEC], sm[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    mn[i] = INFINITY;
    mx[i] = -INFINITY;
    sm[i] = 0.f;
  }
  for (int r = 0; r < n_rows; ++r) {
    Vec<T> x;
    x.load(krow0 + r * ksr + col);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      mn[i] = fminf(mn[i], x.v[i]);
      mx[i] = fmaxf(mx[i], x.v[i]);
      sm[i] += x.v[i];
    }
  }
  const float inv_n = 1.0f / (float)n_rows;
  float mean[VEC], m2[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    mean[i] = sm[i] / (float)n_rows;
    m2[i] = 0.f;
  }
  for (int r = 0; r < n_rows; ++r) {
    Vec<T> x;
    x.load(krow0 + r * ksr + col);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float d = x.v[i] - mean[i];
      m2[i] += d * d;
    }
  }
  Vec<T> o;
#pragma unroll
  for (int i = 0; i < VEC; ++i) o.v[i] = mn[i];
  o.store(smin + col);
#pragma unroll
  for (int i = 0; i < VEC; ++i) o.v[i] = mx[i];
  o.store(smax + col);
#pragma unroll
  for (int i = 0; i < VEC; ++i) o.v[i] = mean[i];
  o.store(smean + col);
#pragma unroll
  for (int i = 0; i < VEC; ++i) o.v[i] = fmaxf(sqrtf(m2[i] * inv_n), 1e-6f);
  o.store(sstd + col);
}

template <typename T, int LPR>
__global__ __launch_bounds__(256) void page_stats_kernel(
    const T* __restrict__ k, int64_t ksb, int64_t ksh, int64_t ksr, StatsPtrs st, int64_t ssb,
    int64_t ssh, int64_t ssp, int Hkv, int seq_len, const int32_t* __restrict__ seq_lens,
    int page_size, int page_begin, int page_end) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int PPW = 256 / LPR;  // pages per workgroup
  const int seg = threadIdx.x / LPR;
  const int col = (threadIdx.x % LPR) * VEC;
  const int page = page_begin + blockIdx.x * PPW + seg;
  if (page >= page_end) return;
  const int bh = blockIdx.y;
  const int b = bh / Hkv, h = bh % Hkv;
  const int r0 = page * page_size;
  const int len = seq_lens ? seq_lens[b] : seq_len;
  const int n_rows = min(page_size, len - r0);
  if (n_rows <= 0) return;
  const T* krow0 = k + b * ksb + h * ksh + (int64_t)r0 * ksr;
  const int64_t so = b * ssb + h * ssh + (int64_t)page * ssp;
  page_stats_one<T, LPR>(krow0, ksr, n_rows, (T*)st.kmin + so, (T*)st.kmax + so,
                         (T*)st.kmean + so, (T*)st.kstd + so, col);
}

// One segment per (b, kv head): write row `pos` of K and V, then recompute the
// statistics of page pos / ps from the cache rows (the new row taken from
// registers).
template <typename T, int LPR>
__global__ __launch_bounds__(64) void append_kernel(
    const T* __restrict__ k_new, const T* __restrict__ v_new, int64_t nsb, int64_t nsh, T* k, T* v,
    int64_t ksb, int64_t ksh, int64_t ksr, StatsPtrs st, int64_t ssb, int64_t ssh, int64_t ssp,
    int B, int Hkv, const int* __restrict__ pos_per_batch, int pos_scalar, int page_size,
    const int32_t* __restrict__ block_table, int64_t btsb, int bt_blocks) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SPB = 64 / LPR;
  const int seg = threadIdx.x / LPR;
  const int col = (threadIdx.x % LPR) * VEC;
  const int bh = blockIdx.x * SPB + seg;
  if (bh >= B * Hkv) return;
  const int b = bh / Hkv, h = bh % Hkv;
  const int pos = pos_per_batch ? pos_per_batch[b] : pos_scalar;
  if (pos < 0) return;
  const T* kn = k_new + b * nsb + h * nsh;
  const T* vn = v_new + b * nsb + h * nsh;
  T* kh = k + b * ksb + h * ksh;
  T* vh = v + b * ksb + h * ksh;
  if (block_table) {
    // every row of this page lies in one block of the pool: kh + r * ksr
    // addresses row r of the page for r in [page * ps, pos]
    const int blk = block_table[b * btsb + pos / page_size];
    if (blk < 0 || blk >= bt_blocks) return;
    const int64_t shift = (int64_t)blk * ksb + h * ksh - (int64_t)(pos / page_size) * page_size * ksr;
    kh = k + shift;
    vh = v + shift;
  }
  const int64_t so = b * ssb + h * ssh + (int64_t)(pos / page_size) * ssp;
  PageStatRows<T> rows{(T*)st.kmin + so, (T*)st.kmax + so, (T*)st.kmean + so, (T*)st.kstd + so};
  append_row<T, LPR>(kn, vn, kh, vh, ksr, pos, page_size, rows, col);
}

template <typename T, int LPR>
int launch_stats(const void* k, int64_t ksb, int64_t ksh, int64_t ksr, StatsPtrs st, int64_t ssb,
                 int64_t ssh, int64_t ssp, int B, int Hkv, int seq_len, const int32_t* seq_lens,
                 int ps, int p0, int p1, hipStream_t s) {
  constexpr int PPW = 256 / LPR;
  dim3 grid((p1 - p0 + PPW - 1) / PPW, B * Hkv);
  hipLaunchKernelGGL((page_stats_kernel<T, LPR>), grid, dim3(256), 0, s, (const T*)k, ksb, ksh,
                     ksr, st, ssb, ssh, ssp, Hkv, seq_len, seq_lens, ps, p0, p1);
  return check_launch("page_stats_kernel");
}

template <typename T, int LPR>
int launch_append(const void* kn, const void* vn, int64_t nsb, int64_t nsh, void* k, void* v,
                  int64_t ksb, int64_t ksh, int64_t ksr, StatsPtrs st, int64_t ssb, int64_t ssh,
                  int64_t ssp, int B, int Hkv, const int* pos_b, int pos, int ps,
                  const int32_t* bt, int64_t btsb, int bt_blocks, hipStream_t s) {
  constexpr int SPB = 64 / LPR;
  dim3 grid((B * Hkv + SPB - 1) / SPB);
  hipLaunchKernelGGL((append_kernel<T, LPR>), grid, dim3(64), 0, s, (const T*)kn, (const T*)vn,
                     nsb, nsh, (T*)k, (T*)v, ksb, ksh, ksr, st, ssb, ssh, ssp, B, Hkv, pos_b, pos,
                     ps, bt, btsb, bt_blocks);
  return check_launch("append_kernel");
}

}  // namespace

extern "C" int ekv_page_stats(const void* k, int64_t k_stride_b, int64_t k_stride_h,
                              int64_t k_stride_row, void* kmin, void* kmax, void* kmean, void* kstd,
                              int64_t s_stride_b, int64_t s_stride_h, int64_t s_stride_page, int B,
                              int Hkv, int D, int seq_len, const int32_t* seq_lens,
                              int page_size, int page_begin, int page_end, int dtype,
                              void* stream) {
  EKV_REQUIRE(k && kmin && kmax && kmean && kstd, "ekv_page_stats: null pointer");
  EKV_REQUIRE(B > 0 && Hkv > 0 && page_size > 0 && seq_len >= 0, "ekv_page_stats: bad sizes");
  EKV_REQUIRE(page_begin >= 0 && page_end >= page_begin, "ekv_page_stats: bad page range");
  EKV_REQUIRE((int64_t)page_end * page_size < (int64_t)seq_len + page_size,
              "ekv_page_stats: page_end %d beyond seq_len %d", page_end, seq_len);
  if (page_end == page_begin) return EKV_OK;
  StatsPtrs st{kmin, kmax, kmean, kstd};
  hipStream_t s = (hipStream_t)stream;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    return dispatch_lpr<T>(D, [&](auto lpr) {
      return launch_stats<T, decltype(lpr)::value>(k, k_stride_b, k_stride_h, k_stride_row, st,
                                                   s_stride_b, s_stride_h, s_stride_page, B, Hkv,
                                                   seq_len, seq_lens, page_size, page_begin,
                                                   page_end, s);
    });
  });
}

extern "C" int ekv_append(const void* k_new, const void* v_new, int64_t new_stride_b,
                          int64_t new_stride_h, void* k, void* v, int64_t k_stride_b,
                          int64_t k_stride_h, int64_t k_stride_row, void* kmin, void* kmax,
                          void* kmean, void* kstd, int64_t s_stride_b, int64_t s_stride_h,
                          int64_t s_stride_page, int B, int Hkv, int D, int pos,
                          const int32_t* pos_per_batch, const int32_t* block_table,
                          int64_t bt_stride_b, int bt_blocks, int page_size, int dtype,
                          void* stream) {
  EKV_REQUIRE(k_new && v_new && k && v && kmin && kmax && kmean && kstd,
              "ekv_append: null pointer");
  EKV_REQUIRE(B > 0 && Hkv > 0 && page_size > 0, "ekv_append: bad sizes");
  EKV_REQUIRE(pos_per_batch || pos >= 0, "ekv_append: negative position");
  EKV_REQUIRE(!block_table || bt_blocks > 0, "ekv_append: a block table needs bt_blocks > 0");
  StatsPtrs st{kmin, kmax, kmean, kstd};
  hipStream_t s = (hipStream_t)stream;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    return dispatch_lpr<T>(D, [&](auto lpr) {
      return launch_append<T, decltype(lpr)::value>(
          k_new, v_new, new_stride_b, new_stride_h, k, v, k_stride_b, k_stride_h, k_stride_row, st,
          s_stride_b, s_stride_h, s_stride_page, B, Hkv, pos_per_batch, pos, page_size,
          block_table, bt_stride_b, bt_blocks, s);
    });
  });
}
