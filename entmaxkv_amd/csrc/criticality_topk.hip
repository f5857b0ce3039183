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
// Page keys staged in LDS by the top-k pass (16384 pages = 256k tokens at
// page size 16, 64 KB); longer caches re-read the scores on every pass.
constexpr int kMaxStagedKeys = 16384;
// Batch * kv heads from which one workgroup per head fills the GPU.
constexpr int kHeadPathMinHeads = 128;

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

// Per-wave counts of two 1-bit flags, combined into block-exclusive prefixes
// with one barrier.  `cnt` needs 2 * (NT / 64) ints.
template <int NT>
__device__ __forceinline__ void block_flag_prefix(bool f0, bool f1, int* cnt, int& pre0, int& pre1,
                                                  int& tot0, int& tot1) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const uint64_t m0 = __ballot(f0), m1 = __ballot(f1);
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  if (lane == 0) {
    cnt[2 * wid] = __popcll(m0);
    cnt[2 * wid + 1] = __popcll(m1);
  }
  __syncthreads();
  int b0 = 0, b1 = 0, t0 = 0, t1 = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) {
    const int c0 = cnt[2 * w], c1 = cnt[2 * w + 1];
    if (w < wid) {
      b0 += c0;
      b1 += c1;
    }
    t0 += c0;
    t1 += c1;
  }
  __syncthreads();
  pre0 = b0 + __popcll(m0 & below);
  pre1 = b1 + __popcll(m1 & below);
  tot0 = t0;
  tot1 = t1;
}

// Block-wide top-k over `num_pages` group keys; writes ascending indices to
// out[0..k) and `last_page` to out[k] when last_page >= 0.  blockDim == NT.
// The keys come from `lds_keys` when `prestaged`, are staged there first when
// they fit (`lds_cap` keys), and are otherwise recomputed from the scores on
// every pass, 8 loads in flight per thread (the scores must be visible to
// this workgroup: written by a previous launch or by this workgroup).  Radix select: 8 bits per pass
// from the top, then one pack pass.
template <typename T, int G, int NT = kThreads>
__device__ void topk_select_block(const T* __restrict__ s0, int64_t head_stride, int num_pages,
                                  int k, int last_page, int32_t* __restrict__ out,
                                  uint32_t* lds_keys, int lds_cap, bool prestaged = false) {
  __shared__ unsigned hist[256];
  __shared__ int scan_scratch[NT / 64 + 1];
  __shared__ int flag_cnt[2 * (NT / 64)];
  __shared__ int sel_bin, sel_kk;
  const int tid = threadIdx.x;
  constexpr int kBatch = 8;
  constexpr int kThreads = NT;
  k = min(k, num_pages);
  const bool staged = prestaged || num_pages <= lds_cap;
  // group key of page p: the maximum over the group's query heads
  auto gkey = [&](int p) -> uint32_t {
    uint32_t kk = ScoreKey<T>::key(s0[p]);
#pragma unroll
    for (int g = 1; g < G; ++g) kk = max(kk, ScoreKey<T>::key(s0[g * head_stride + p]));
    return kk;
  };
  if (staged && !prestaged) {
    for (int p0 = 0; p0 < num_pages; p0 += kThreads * kBatch) {
      uint32_t kv[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int p = p0 + j * kThreads + tid;
        kv[j] = p < num_pages ? gkey(p) : 0u;
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int p = p0 + j * kThreads + tid;
        if (p < num_pages) lds_keys[p] = kv[j];
      }
    }
    __syncthreads();
  }
  // visits every page key (from LDS when staged) with f(p, key)
  auto for_keys = [&](auto&& f) {
    for (int p0 = 0; p0 < num_pages; p0 += kThreads * kBatch) {
      uint32_t kv[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int p = p0 + j * kThreads + tid;
        kv[j] = p < num_pages ? (staged ? lds_keys[p] : gkey(p)) : 0u;
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int p = p0 + j * kThreads + tid;
        if (p < num_pages) f(p, kv[j]);
      }
    }
  };

  uint32_t thr = 0;
  int kk = 0;  // how many pages with key == thr to take
  const bool take_all = (k == num_pages);
  if (k > 0 && !take_all) {
    uint32_t prefix = 0, pmask = 0;
    kk = k;
    for (int shift = ScoreKey<T>::kBits - 8; shift >= 0; shift -= 8) {
      if (tid < 256) hist[tid] = 0;
      __syncthreads();
      for_keys([&](int, uint32_t key) {
        if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
      });
      __syncthreads();
      const int bin = 255 - tid;  // thread t < 256 owns bin 255 - t: scan from the top
      const int c = tid < 256 ? (int)hist[bin] : 0;
      int tot;
      const int above = block_excl_scan(c, scan_scratch, &tot);
      if (tid < 256 && above < kk && above + c >= kk) {
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
    // every key > thr is taken, and the first kk keys == thr in page order
    int gt_base = 0, eq_base = 0;
    for (int c0 = 0; c0 < num_pages; c0 += kThreads) {
      const int p = c0 + tid;
      bool gt = false, eq = false;
      if (p < num_pages) {
        if (take_all) {
          gt = true;
        } else {
          const uint32_t key = staged ? lds_keys[p] : gkey(p);
          gt = key > thr;
          eq = key == thr;
        }
      }
      int gt_pre, eq_pre, gt_tot, eq_tot;
      block_flag_prefix<NT>(gt, eq, flag_cnt, gt_pre, eq_pre, gt_tot, eq_tot);
      const int eq_rank = eq_base + eq_pre;
      if (gt || (eq && eq_rank < kk)) out[gt_base + gt_pre + min(eq_rank, kk)] = p;
      gt_base += gt_tot;
      eq_base += eq_tot;
    }
  }
  if (tid == 0 && last_page >= 0) out[k] = last_page;
}

// One workgroup of kHeadThreads per (b, kv head): scores every page of the
// head (16-byte loads, kHeadUnroll pages per row segment in flight), keeps
// the group-max keys in LDS and, when k_sel >= 0, selects the top-k pages in
// the same workgroup.  No cross-workgroup communication.
constexpr int kHeadThreads = 512;
constexpr int kHeadUnroll = 8;

template <typename T, int LPR, int G, int U>
__global__ __launch_bounds__(kHeadThreads) void criticality_head_kernel(
    const T* __restrict__ q, int64_t qsb, int64_t qsh, const T* __restrict__ kmin,
    const T* __restrict__ kmax, int64_t ssb, int64_t ssh, int64_t ssp,
    const float* __restrict__ slopes, T* __restrict__ scores, int H, int Hkv, int num_pages,
    int page_size, int seq_len, int q_pos, int k_sel, int last_page, int32_t* page_indices,
    int64_t pisb, int64_t pish, int lds_key_cap) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SEGS = kHeadThreads / LPR;
  constexpr int ROUND = SEGS * U;
  extern __shared__ uint32_t lds_keys[];
  const int seg = threadIdx.x / LPR;
  const int sl = threadIdx.x % LPR;
  const int col = sl * VEC;
  const int bkv = blockIdx.x;
  const int b = bkv / Hkv, kvh = bkv % Hkv;
  const int h0 = kvh * G;
  const bool keep_keys = k_sel >= 0 && num_pages <= lds_key_cap;

  // q in its storage format plus a per-element "q >= 0" mask: the bound of
  // element d is kmax where q_d >= 0 and kmin elsewhere (kernels/page_criticality.py:88-95)
  uint4 qraw[G], qmask[G];
  float slope[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    qraw[g] = ld16(q + b * qsb + (h0 + g) * qsh + col);
    qmask[g] = Dot16<T>::nonneg_mask(qraw[g]);
    slope[g] = slopes ? slopes[h0 + g] : 0.f;
  }
  const T* kmn = kmin + b * ssb + kvh * ssh;
  const T* kmx = kmax + b * ssb + kvh * ssh;
  T* sbase = scores + ((int64_t)b * H + h0) * num_pages;

  for (int p0 = 0; p0 < num_pages; p0 += ROUND) {
    uint4 lo[U], hi[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = p0 + u * SEGS + seg;
      if (p < num_pages) {
        lo[u] = ld16(kmn + (int64_t)p * ssp + col);
        hi[u] = ld16(kmx + (int64_t)p * ssp + col);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = p0 + u * SEGS + seg;
      uint32_t key = 0;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = Dot16<T>::dot(qraw[g], bit_select(lo[u], hi[u], qmask[g]), 0.f);
        acc = seg_sum<LPR>(acc);
        if (slopes) {
          const int last_pos = min((p + 1) * page_size - 1, seq_len - 1);
          acc = add_rn(acc, mul_rn(slope[g], (float)(last_pos - q_pos)));
        }
        const T sv = from_f<T>(acc);
        key = max(key, ScoreKey<T>::key(sv));
        if (p < num_pages && sl == 0) sbase[(int64_t)g * num_pages + p] = sv;
      }
      if (keep_keys && p < num_pages && sl == 0) lds_keys[p] = key;
    }
  }
  if (k_sel < 0) return;
  __syncthreads();
  topk_select_block<T, G, kHeadThreads>(sbase, num_pages, num_pages, k_sel, last_page,
                                               page_indices + b * pisb + kvh * pish, lds_keys,
                                               keep_keys ? num_pages : 0, keep_keys);
}

template <typename T, int LPR, int G>
__global__ __launch_bounds__(kThreads) void criticality_kernel(
    const T* __restrict__ q, int64_t qsb, int64_t qsh, const T* __restrict__ kmin,
    const T* __restrict__ kmax, int64_t ssb, int64_t ssh, int64_t ssp,
    const float* __restrict__ slopes, T* __restrict__ scores, int H, int Hkv, int num_pages,
    int page_size, int seq_len, int q_pos) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SEGS = kThreads / LPR;
  const int seg = threadIdx.x / LPR;
  const int sl = threadIdx.x % LPR;
  const int col = sl * VEC;
  const int bkv = blockIdx.y;
  const int b = bkv / Hkv, kvh = bkv % Hkv;
  const int h0 = kvh * G;
  uint4 qraw[G], qmask[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    qraw[g] = ld16(q + b * qsb + (h0 + g) * qsh + col);
    qmask[g] = Dot16<T>::nonneg_mask(qraw[g]);
  }
  const T* kmn = kmin + b * ssb + kvh * ssh;
  const T* kmx = kmax + b * ssb + kvh * ssh;
  const int p_base = blockIdx.x * (SEGS * kUnroll) + seg;
  uint4 lo[kUnroll], hi[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int p = p_base + u * SEGS;
    if (p < num_pages) {
      lo[u] = ld16(kmn + (int64_t)p * ssp + col);
      hi[u] = ld16(kmx + (int64_t)p * ssp + col);
    }
  }
  T* sbase = scores + ((int64_t)b * H + h0) * num_pages;
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int p = p_base + u * SEGS;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float acc = Dot16<T>::dot(qraw[g], bit_select(lo[u], hi[u], qmask[g]), 0.f);
      acc = seg_sum<LPR>(acc);
      if (p < num_pages && sl == 0) {
        if (slopes) {
          const int last_pos = min((p + 1) * page_size - 1, seq_len - 1);
          acc = add_rn(acc, mul_rn(slopes[h0 + g], (float)(last_pos - q_pos)));
        }
        sbase[(int64_t)g * num_pages + p] = from_f<T>(acc);
      }
    }
  }
}

template <typename T, int G>
__global__ __launch_bounds__(kThreads) void topk_kernel(const T* __restrict__ scores, int H, int Hkv,
                                                        int num_pages, int k, int last_page,
                                                        int32_t* page_indices, int64_t pisb,
                                                        int64_t pish, int lds_key_cap) {
  const int bkv = blockIdx.x;
  const int b = bkv / Hkv, kvh = bkv % Hkv;
  const T* s0 = scores + ((int64_t)b * H + kvh * G) * num_pages;
  extern __shared__ uint32_t lds_keys[];
  topk_select_block<T, G, kThreads>(s0, num_pages, num_pages, k, last_page,
                                           page_indices + b * pisb + kvh * pish, lds_keys,
                                           lds_key_cap);
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
                                    int64_t pi_stride_b, int64_t pi_stride_h, int dtype,
                                    void* stream) {
  EKV_REQUIRE(q && kmin && kmax && scores, "ekv_page_criticality: null pointer");
  EKV_REQUIRE(B > 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "ekv_page_criticality: bad head counts");
  EKV_REQUIRE(num_pages >= 0 && page_size > 0, "ekv_page_criticality: bad page counts");
  EKV_REQUIRE(k_select < 0 || page_indices, "ekv_page_criticality: top-k needs page_indices");
  // an empty page range is handled by the caller (the page table is just the sentinel)
  EKV_REQUIRE(num_pages > 0, "ekv_page_criticality: no pages to score");
  hipStream_t s = (hipStream_t)stream;
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    return dispatch_lpr<T>(D, [&](auto lpr) {
      constexpr int LPR = decltype(lpr)::value;
      return dispatch_group(H / Hkv, [&](auto gv) {
        constexpr int G = decltype(gv)::value;
        if (B * Hkv >= kHeadPathMinHeads) {
          // one workgroup per (b, kv head), top-k in the same launch
          const int cap = (k_select >= 0 && num_pages <= kMaxStagedKeys) ? num_pages : 0;
          constexpr int U = G >= 8 ? 2 : 16 / G;
          hipLaunchKernelGGL((criticality_head_kernel<T, LPR, G, U>), dim3(B * Hkv),
                             dim3(kHeadThreads), (size_t)cap * sizeof(uint32_t), s, (const T*)q,
                             q_stride_b, q_stride_h, (const T*)kmin, (const T*)kmax, s_stride_b,
                             s_stride_h, s_stride_page, alibi_slopes, (T*)scores, H, Hkv, num_pages,
                             page_size, seq_len, q_pos, k_select, last_page, page_indices,
                             pi_stride_b, pi_stride_h, cap);
          return check_launch("criticality_head_kernel");
        }
        // few heads: spread the pages of each head over many workgroups, then
        // select in a second launch
        constexpr int PPW = (kThreads / LPR) * kUnroll;
        dim3 grid((num_pages + PPW - 1) / PPW, B * Hkv);
        hipLaunchKernelGGL((criticality_kernel<T, LPR, G>), grid, dim3(kThreads), 0, s, (const T*)q,
                           q_stride_b, q_stride_h, (const T*)kmin, (const T*)kmax, s_stride_b,
                           s_stride_h, s_stride_page, alibi_slopes, (T*)scores, H, Hkv, num_pages,
                           page_size, seq_len, q_pos);
        if (k_select >= 0) {
          int rc = check_launch("criticality_kernel");
          if (rc) return rc;
          const int cap2 = num_pages <= kMaxStagedKeys ? num_pages : 0;
          hipLaunchKernelGGL((topk_kernel<T, G>), dim3(B * Hkv), dim3(kThreads),
                             (size_t)cap2 * sizeof(uint32_t), s, (const T*)scores, H, Hkv,
                             num_pages, k_select, last_page, page_indices, pi_stride_b,
                             pi_stride_h, cap2);
          return check_launch("topk_kernel");
        }
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
      const int cap = num_pages <= kMaxStagedKeys ? num_pages : 0;
      hipLaunchKernelGGL((topk_kernel<T, G>), dim3(B * Hkv), dim3(kThreads),
                         (size_t)cap * sizeof(uint32_t), s, (const T*)scores, H, Hkv, num_pages, k,
                         last_page, page_indices, pi_stride_b, pi_stride_h, cap);
      return check_launch("topk_kernel");
    });
  });
}
