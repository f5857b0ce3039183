// Page criticality scoring and top-k page selection.
//
// criticality: score[b, h, p] = sum_d max(q_d * kmin_pd, q_d * kmax_pd)
//   (+ fp32 ALiBi bonus), fp32 accumulation, stored in the query dtype.
//   Follows kernels/page_criticality.py:24-104,142-187 (scale 1.0).
// top-k: per (b, kv head) the k pages with the largest score (under GQA the
//   group maximum of the query heads' scores), packed in ascending page order,
//   ties broken toward the lower page index, followed by the last-page
//   sentinel.  Replaces torch.topk + the index buffer of attention_topk.py:52-71
//   and kv_cache.py:167-185.
//
// Layout: one workgroup (256 threads) scores PAGES_PER_WG pages of one
// (b, kv head); a row segment of LPR lanes owns one page and loads its kmin
// and kmax rows with 16-byte loads.  Every page is read once for all G query
// heads of the group.  When top-k is fused, the last workgroup of a
// (b, kv head) to finish runs a block-wide radix select over the page scores
// (already resident in L2) and writes the page table.
#include "ekv_common.h"
#include "../../include/entmaxkv.h"

using namespace ekv;

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;  // pages per segment per workgroup

// Order-preserving unsigned key of a stored score; NaN maps to the top.
template <typename T> struct ScoreKey;
template <> struct ScoreKey<_Float16> {
  static constexpr int kBits = 16;
  static __device__ __forceinline__ uint32_t key(_Float16 x) {
    uint16_t u = __builtin_bit_cast(uint16_t, x);
    if ((u & 0x7fffu) > 0x7c00u) return 0xffffu;
    return (u & 0x8000u) ? (uint32_t)(~u & 0xffffu) : (uint32_t)(u | 0x8000u);
  }
};
template <> struct ScoreKey<bf16_t> {
  static constexpr int kBits = 16;
  static __device__ __forceinline__ uint32_t key(bf16_t x) {
    uint16_t u = x.bits;
    if ((u & 0x7fffu) > 0x7f80u) return 0xffffu;
    return (u & 0x8000u) ? (uint32_t)(~u & 0xffffu) : (uint32_t)(u | 0x8000u);
  }
};
template <> struct ScoreKey<float> {
  static constexpr int kBits = 32;
  static __device__ __forceinline__ uint32_t key(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0xffffffffu;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  }
};

template <typename T, int G>
__device__ __forceinline__ uint32_t group_key(const T* __restrict__ s0, int64_t head_stride, int p) {
  uint32_t k = ScoreKey<T>::key(s0[p]);
#pragma unroll
  for (int g = 1; g < G; ++g) k = max(k, ScoreKey<T>::key(s0[g * head_stride + p]));
  return k;
}

// Block-wide top-k over `num_pages` group keys; writes ascending indices to
// out[0..k) and `last_page` to out[k] when last_page >= 0.  blockDim == 256.
template <typename T, int G>
__device__ void topk_select_block(const T* __restrict__ s0, int64_t head_stride, int num_pages,
                                  int k, int last_page, int32_t* __restrict__ out) {
  __shared__ unsigned hist[256];
  __shared__ int scan_scratch[kThreads / 64 + 1];
  __shared__ int sel_bin, sel_kk;
  const int tid = threadIdx.x;
  k = min(k, num_pages);
  uint32_t thr = 0;
  int kk = 0;  // how many pages with key == thr to take
  const bool take_all = (k == num_pages);
  if (k > 0 && !take_all) {
    uint32_t prefix = 0, pmask = 0;
    kk = k;
    for (int shift = ScoreKey<T>::kBits - 8; shift >= 0; shift -= 8) {
      hist[tid] = 0;
      __syncthreads();
      for (int p = tid; p < num_pages; p += kThreads) {
        uint32_t key = group_key<T, G>(s0, head_stride, p);
        if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      }
      __syncthreads();
      const int bin = 255 - tid;  // thread t owns bin 255 - t: scan from the top
      const int c = (int)hist[bin];
      int tot;
      const int above = block_excl_scan(c, scan_scratch, &tot);
      if (above < kk && above + c >= kk) {
        sel_bin = bin;
        sel_kk = kk - above;
      }
      __syncthreads();
      prefix |= ((uint32_t)sel_bin) << shift;
      pmask |= 255u << shift;
      kk = sel_kk;
      __syncthreads();
    }
    thr = prefix;
  }
  if (k > 0) {
    int base = 0, eq_base = 0;
    for (int c0 = 0; c0 < num_pages; c0 += kThreads) {
      const int p = c0 + tid;
      bool gt = false, eq = false;
      if (p < num_pages) {
        if (take_all) {
          gt = true;
        } else {
          uint32_t key = group_key<T, G>(s0, head_stride, p);
          gt = key > thr;
          eq = key == thr;
        }
      }
      int eq_tot, tot;
      const int eq_rank = block_excl_scan(eq ? 1 : 0, scan_scratch, &eq_tot);
      const bool take = gt || (eq && eq_base + eq_rank < kk);
      const int pos = block_excl_scan(take ? 1 : 0, scan_scratch, &tot);
      if (take) out[base + pos] = p;
      base += tot;
      eq_base += eq_tot;
    }
  }
  if (tid == 0 && last_page >= 0) out[k] = last_page;
}

template <typename T, int LPR, int G>
__global__ __launch_bounds__(kThreads) void criticality_kernel(
    const T* __restrict__ q, int64_t qsb, int64_t qsh, const T* __restrict__ kmin,
    const T* __restrict__ kmax, int64_t ssb, int64_t ssh, int64_t ssp,
    const float* __restrict__ slopes, T* __restrict__ scores, int H, int Hkv, int num_pages,
    int page_size, int seq_len, int q_pos, int k_sel, int last_page, int32_t* page_indices,
    int64_t pisb, int64_t pish, int* counters) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SEGS = kThreads / LPR;
  const int seg = threadIdx.x / LPR;
  const int col = (threadIdx.x % LPR) * VEC;
  const int bkv = blockIdx.y;
  const int b = bkv / Hkv, kvh = bkv % Hkv;
  const int h0 = kvh * G;

  float qv[G][VEC];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    Vec<T> x;
    x.load(q + b * qsb + (h0 + g) * qsh + col);
#pragma unroll
    for (int i = 0; i < VEC; ++i) qv[g][i] = x.v[i];
  }
  const T* kmn = kmin + b * ssb + kvh * ssh;
  const T* kmx = kmax + b * ssb + kvh * ssh;
  const int p_base = blockIdx.x * (SEGS * kUnroll) + seg;

  VecRaw<T> lo[kUnroll], hi[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int p = p_base + u * SEGS;
    if (p < num_pages) {
      lo[u].load(kmn + (int64_t)p * ssp + col);
      hi[u].load(kmx + (int64_t)p * ssp + col);
    }
  }
  T* sbase = scores + ((int64_t)b * H + h0) * num_pages;
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int p = p_base + u * SEGS;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const float qi = qv[g][i];
        acc += qi * (qi >= 0.f ? hi[u].get(i) : lo[u].get(i));
      }
      acc = seg_sum<LPR>(acc);
      if (p < num_pages && (threadIdx.x % LPR) == 0) {
        if (slopes) {
          const int last_pos = min((p + 1) * page_size - 1, seq_len - 1);
          const float bonus = mul_rn(slopes[h0 + g], (float)(last_pos - q_pos));
          acc = add_rn(acc, bonus);
        }
        sbase[(int64_t)g * num_pages + p] = from_f<T>(acc);
      }
    }
  }
  if (k_sel < 0) return;
  if (!last_arrival(&counters[bkv], gridDim.x)) return;
  topk_select_block<T, G>(sbase, num_pages, num_pages, k_sel, last_page,
                          page_indices + b * pisb + kvh * pish);
}

template <typename T, int G>
__global__ __launch_bounds__(kThreads) void topk_kernel(const T* __restrict__ scores, int H, int Hkv,
                                                        int num_pages, int k, int last_page,
                                                        int32_t* page_indices, int64_t pisb,
                                                        int64_t pish) {
  const int bkv = blockIdx.x;
  const int b = bkv / Hkv, kvh = bkv % Hkv;
  const T* s0 = scores + ((int64_t)b * H + kvh * G) * num_pages;
  topk_select_block<T, G>(s0, num_pages, num_pages, k, last_page,
                          page_indices + b * pisb + kvh * pish);
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

extern "C" int ekv_page_criticality(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                    const void* kmin, const void* kmax, int64_t s_stride_b,
                                    int64_t s_stride_h, int64_t s_stride_page,
                                    const float* alibi_slopes, void* scores, int B, int H, int Hkv,
                                    int D, int num_pages, int page_size, int seq_len, int q_pos,
                                    int k_select, int last_page, int32_t* page_indices,
                                    int64_t pi_stride_b, int64_t pi_stride_h, int32_t* counters,
                                    int dtype, void* stream) {
  EKV_REQUIRE(q && kmin && kmax && scores, "ekv_page_criticality: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "ekv_page_criticality: bad head counts");
  EKV_REQUIRE(num_pages >= 0 && page_size > 0, "ekv_page_criticality: bad page counts");
  EKV_REQUIRE(k_select < 0 || (page_indices && counters),
              "ekv_page_criticality: fused top-k needs page_indices and counters");
  // an empty page range is handled by the caller (the page table is just the sentinel)
  EKV_REQUIRE(num_pages > 0, "ekv_page_criticality: no pages to score");
  hipStream_t s = (hipStream_t)stream;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    return dispatch_lpr<T>(D, [&](auto lpr) {
      constexpr int LPR = decltype(lpr)::value;
      return dispatch_group(H / Hkv, [&](auto gv) {
        constexpr int G = decltype(gv)::value;
        constexpr int PPW = (kThreads / LPR) * kUnroll;
        dim3 grid((num_pages + PPW - 1) / PPW, B * Hkv);
        hipLaunchKernelGGL((criticality_kernel<T, LPR, G>), grid, dim3(kThreads), 0, s,
                           (const T*)q, q_stride_b, q_stride_h, (const T*)kmin, (const T*)kmax,
                           s_stride_b, s_stride_h, s_stride_page, alibi_slopes, (T*)scores, H, Hkv,
                           num_pages, page_size, seq_len, q_pos, k_select, last_page, page_indices,
                           pi_stride_b, pi_stride_h, counters);
        return check_launch("criticality_kernel");
      });
    });
  });
}

extern "C" int ekv_topk_pages(const void* scores, int B, int H, int Hkv, int num_pages, int k,
                              int last_page, int32_t* page_indices, int64_t pi_stride_b,
                              int64_t pi_stride_h, int dtype, void* stream) {
  EKV_REQUIRE(scores && page_indices, "ekv_topk_pages: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "ekv_topk_pages: bad head counts");
  EKV_REQUIRE(num_pages > 0 && k >= 0 && k <= num_pages, "ekv_topk_pages: bad k %d of %d", k,
              num_pages);
  hipStream_t s = (hipStream_t)stream;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    return dispatch_group(H / Hkv, [&](auto gv) {
      constexpr int G = decltype(gv)::value;
      hipLaunchKernelGGL((topk_kernel<T, G>), dim3(B * Hkv), dim3(kThreads), 0, s, (const T*)scores,
                         H, Hkv, num_pages, k, last_page, page_indices, pi_stride_b, pi_stride_h);
      return check_launch("topk_kernel");
    });
  });
}
