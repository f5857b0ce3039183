// Page criticality scoring and top-k page selection.
//
// criticality: score[b, h, p] = sum_d max(q_d * kmin_pd, q_d * kmax_pd)
//   (+ fp32 ALiBi bonus), fp32 accumulation, stored in the query dtype.
//   Follows kernels/page_criticality.py:24-104,142-187 (scale 1.0).
// top-k: per (b, kv head) the k pages with the largest score (under GQA the
//   k pages of best rank over the query heads' own orders, ties to the lower
//   page index), packed in ascending page order, ties broken toward the lower
//   page index, followed by the last-page sentinel.  Replaces torch.topk + the index buffer of attention_topk.py:52-71
//   and kv_cache.py:167-185.
//
// Ragged batches (seq_lens non-null): every (b, kv head) scores, selects and
// appends the sentinel for its own length (ragged_topk, topk_device.h);
// `num_pages` is then the score row stride (the longest sequence).
//
// Layout: with B * Hkv >= 128, one workgroup per (b, kv head) scores every
// page of the head and selects its top-k in the same launch
// (criticality_head_kernel); otherwise each head's pages are spread over
// workgroups of 256 threads (criticality_kernel) and a second launch selects
// (topk_kernel).  A row segment of LPR lanes owns one page and loads its kmin
// and kmax rows with 16-byte loads; every page is read once for all G query
// heads of the group.
#include "ekv_common.h"

#ifdef EKV_PHASE_TIMERS
__device__ unsigned long long ekv_crit_timers[4096 * 8];
#define EKV_CSTAMP(i) \
  if (threadIdx.x == 0 && blockIdx.x < 4096) ekv_crit_timers[blockIdx.x * 8 + (i)] = wall_clock64()
extern "C" int ekv_debug_crit_timers(unsigned long long* host, int n) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(ekv_crit_timers), n * sizeof(unsigned long long));
}
#endif

#include "topk_device.h"
#include "../../include/entmaxkv.h"

using namespace ekv;

namespace {

using namespace ekv::topk;

// One workgroup of kHeadThreads per (b, kv head): scores every page of the
// head (16-byte loads, kHeadUnroll pages per row segment in flight), keeps
// the page keys in LDS (G == 1) and, when k_sel >= 0, selects the top-k pages in
// the same workgroup.  No cross-workgroup communication.
constexpr int kHeadThreads = 512;
constexpr int kHeadUnroll = 8;

template <typename T, int LPR, int G, int U>
__global__ __launch_bounds__(kHeadThreads) void criticality_head_kernel(
    const T* __restrict__ q, int64_t qsb, int64_t qsh, const T* __restrict__ kmin,
    const T* __restrict__ kmax, int64_t ssb, int64_t ssh, int64_t ssp,
    const float* __restrict__ slopes, T* __restrict__ scores, int H, int Hkv, int stride,
    int page_size, int seq_len, int q_pos, int k_sel, int last_page,
    const int32_t* __restrict__ seq_lens, int32_t* page_indices, int64_t pisb, int64_t pish,
    int lds_key_cap, int list_words) {
  extern __shared__ __attribute__((aligned(16))) uint32_t lds_keys[];
  const int bkv = blockIdx.x;
  const int b = bkv / Hkv, kvh = bkv % Hkv;
  const Ragged r = ragged_topk(seq_lens, b, page_size, stride, seq_len, q_pos, k_sel, last_page);
  // G > 1 keeps its page ranks and candidate list in LDS instead of keys
  const bool keep_keys = G == 1 && r.k >= 0 && r.count <= lds_key_cap;
  EKV_CSTAMP(0);
  T* sbase = criticality_scan_head<T, LPR, G, kHeadThreads, U>(
      q, qsb, qsh, kmin, kmax, ssb, ssh, ssp, slopes, scores, H, stride, r.count, page_size,
      r.seq_len, r.q_pos, b, kvh, keep_keys ? lds_keys : nullptr);
  if (r.k < 0) return;
  __syncthreads();
  EKV_CSTAMP(1);
  topk_select_block<T, G, kHeadThreads>(sbase, stride, r.count, r.k, r.last_page,
                                        page_indices + b * pisb + kvh * pish, lds_keys,
                                        G > 1 ? lds_key_cap : (keep_keys ? r.count : 0),
                                        keep_keys, nullptr, lds_keys + stride, nullptr, 0,
                                        list_words);
}

template <typename T, int LPR, int G>
__global__ __launch_bounds__(kThreads) void criticality_kernel(
    const T* __restrict__ q, int64_t qsb, int64_t qsh, const T* __restrict__ kmin,
    const T* __restrict__ kmax, int64_t ssb, int64_t ssh, int64_t ssp,
    const float* __restrict__ slopes, T* __restrict__ scores, int H, int Hkv, int stride,
    int page_size, int seq_len_all, int q_pos_all, const int32_t* __restrict__ seq_lens,
    int rev, int nt) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SEGS = kThreads / LPR;
  // rev: the workgroups take their (b, kv head, page round) in the opposite
  // order of their dispatch, last first
  const int lin = blockIdx.y * gridDim.x + blockIdx.x;
  const int wg = rev ? gridDim.x * gridDim.y - 1 - lin : lin;
  const int wx = wg % gridDim.x;
  const int seg = threadIdx.x / LPR;
  const int sl = threadIdx.x % LPR;
  const int col = sl * VEC;
  const int bkv = wg / gridDim.x;
  const int b = bkv / Hkv, kvh = bkv % Hkv;
  const int h0 = kvh * G;
  const Ragged r = ragged_topk(seq_lens, b, page_size, stride, seq_len_all, q_pos_all, -1, -1);
  const int num_pages = r.count, seq_len = r.seq_len, q_pos = r.q_pos;
  uint4 qraw[G], qmask[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    qraw[g] = ld16(q + b * qsb + (h0 + g) * qsh + col);
    qmask[g] = Dot16<T>::nonneg_mask(qraw[g]);
  }
  const T* kmn = kmin + b * ssb + kvh * ssh;
  const T* kmx = kmax + b * ssb + kvh * ssh;
  const int p_base = wx * (SEGS * kUnroll) + seg;
  if (wx * (SEGS * kUnroll) >= num_pages) return;  // past this sequence's pages
  // unconditional loads (a page past the end re-reads the last one, its
  // result is discarded) so that all of them are in flight together
  uint4 lo[kUnroll], hi[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int p = min(p_base + u * SEGS, num_pages - 1);
    lo[u] = ld16_sel(kmn + (int64_t)p * ssp + col, nt);
    hi[u] = ld16_sel(kmx + (int64_t)p * ssp + col, nt);
  }
  T* sbase = scores + ((int64_t)b * H + h0) * stride;
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
        sbase[(int64_t)g * stride + p] = from_f<T>(acc);
      }
    }
  }
}

template <typename T, int G>
__global__ __launch_bounds__(kThreads) void topk_kernel(const T* __restrict__ scores, int H, int Hkv,
                                                        int stride, int k, int last_page,
                                                        int page_size,
                                                        const int32_t* __restrict__ seq_lens,
                                                        int32_t* page_indices, int64_t pisb,
                                                        int64_t pish, int lds_key_cap,
                                                        int list_words) {
  const int bkv = blockIdx.x;
  const int b = bkv / Hkv, kvh = bkv % Hkv;
  const Ragged r = ragged_topk(seq_lens, b, page_size, stride, 0, 0, k, last_page);
  const T* s0 = scores + ((int64_t)b * H + kvh * G) * stride;
  extern __shared__ __attribute__((aligned(16))) uint32_t lds_keys[];
  topk_select_block<T, G, kThreads>(s0, stride, r.count, r.k, r.last_page,
                                    page_indices + b * pisb + kvh * pish, lds_keys, lds_key_cap,
                                    false, nullptr, lds_keys + stride, nullptr, 0, list_words);
}

// Dynamic LDS of the top-k select over `num_pages` pages: the staged keys
// (G == 1, when they fit) or the page ranks plus the candidate lists (G > 1,
// required: all G lists when they fit, else one).  Returns the bytes (0:
// none) or -1 when a G > 1 select does not fit; `cap` receives the key
// capacity and `list_words` the list words.
int64_t select_lds_bytes(int G, int num_pages, int k, int* cap, int* list_words) {
  *list_words = 0;
  if (G == 1) {
    *cap = num_pages <= kMaxStagedKeys ? num_pages : 0;
    return (int64_t)*cap * 4;
  }
  *cap = num_pages;
  if (num_pages > kMaxStagedKeys) return -1;
  // what the static LDS of these kernels leaves (their group histograms)
  const int64_t limit = kLdsPerWorkgroup - kSelectStaticLds;
  for (bool concurrent : {true, false}) {
    const int64_t bytes = ((int64_t)num_pages + group_list_words(G, k, concurrent)) * 4;
    if (bytes <= limit) {
      *list_words = group_list_words(G, k, concurrent);
      return bytes;
    }
  }
  return -1;
}

int set_lds(const void* kern, int64_t bytes, const char* what) {
  if (bytes <= 65536) return EKV_OK;
  const hipError_t e =
      hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess)
    return set_error(EKV_ERR_HIP, "%s LDS %lld: %s", what, (long long)bytes, hipGetErrorString(e));
  return EKV_OK;
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
                                    int k_select, int last_page, const int32_t* seq_lens,
                                    int32_t* page_indices, int64_t pi_stride_b,
                                    int64_t pi_stride_h, int dtype, void* stream) {
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
        int cap = 0, list_words = 0;
        int64_t sel_lds = 0;
        if (k_select >= 0) {
          sel_lds = select_lds_bytes(G, num_pages, k_select, &cap, &list_words);
          EKV_REQUIRE(sel_lds >= 0,
                      "ekv_page_criticality: group top-k of %d of %d pages does not fit LDS",
                      k_select, num_pages);
        }
        if (one_workgroup_per_head(B * Hkv, seq_lens != nullptr)) {
          // one workgroup per (b, kv head), top-k in the same launch
          constexpr int U = G >= 8 ? 2 : 16 / G;
          auto kern = criticality_head_kernel<T, LPR, G, U>;
          if (int rc = set_lds((const void*)kern, sel_lds, "criticality_head_kernel")) return rc;
          hipLaunchKernelGGL(kern, dim3(B * Hkv), dim3(kHeadThreads), (size_t)sel_lds, s,
                             (const T*)q,
                             q_stride_b, q_stride_h, (const T*)kmin, (const T*)kmax, s_stride_b,
                             s_stride_h, s_stride_page, alibi_slopes, (T*)scores, H, Hkv, num_pages,
                             page_size, seq_len, q_pos, k_select, last_page, seq_lens,
                             page_indices, pi_stride_b, pi_stride_h, cap, list_words);
          return check_launch("criticality_head_kernel");
        }
        // few heads: spread the pages of each head over many workgroups, then
        // select in a second launch
        constexpr int PPW = (kThreads / LPR) * kUnroll;
        dim3 grid((num_pages + PPW - 1) / PPW, B * Hkv);
        hipLaunchKernelGGL((criticality_kernel<T, LPR, G>), grid, dim3(kThreads), 0, s, (const T*)q,
                           q_stride_b, q_stride_h, (const T*)kmin, (const T*)kmax, s_stride_b,
                           s_stride_h, s_stride_page, alibi_slopes, (T*)scores, H, Hkv, num_pages,
                           page_size, seq_len, q_pos, seq_lens, next_scan_order(),
                           stream_nt(B, Hkv, num_pages, D, dtype));
        if (k_select >= 0) {
          int rc = check_launch("criticality_kernel");
          if (rc) return rc;
          auto kern = topk_kernel<T, G>;
          if ((rc = set_lds((const void*)kern, sel_lds, "topk_kernel"))) return rc;
          hipLaunchKernelGGL(kern, dim3(B * Hkv), dim3(kThreads), (size_t)sel_lds, s,
                             (const T*)scores, H, Hkv, num_pages, k_select, last_page, page_size,
                             seq_lens, page_indices, pi_stride_b, pi_stride_h, cap, list_words);
          return check_launch("topk_kernel");
        }
        return check_launch("criticality_kernel");
      });
    });
  });
}

// criticality_split_scores (declared in topk_device.h): criticality_kernel only.
namespace ekv {
namespace topk {
int criticality_split_scores(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                             const void* kmin, const void* kmax, int64_t s_stride_b,
                             int64_t s_stride_h, int64_t s_stride_page,
                             const float* alibi_slopes, void* scores, int B, int H, int Hkv,
                             int D, int num_pages, int page_size, int seq_len, int q_pos,
                             const int32_t* seq_lens, int dtype, hipStream_t s, int rev,
                             int nt) {
  return dispatch_dtype(dtype, [&](auto tv) {
    using T = decltype(tv);
    return dispatch_lpr<T>(D, [&](auto lpr) {
      constexpr int LPR = decltype(lpr)::value;
      return dispatch_group(H / Hkv, [&](auto gv) {
        constexpr int G = decltype(gv)::value;
        constexpr int PPW = (kThreads / LPR) * kUnroll;
        dim3 grid((num_pages + PPW - 1) / PPW, B * Hkv);
        hipLaunchKernelGGL((criticality_kernel<T, LPR, G>), grid, dim3(kThreads), 0, s,
                           (const T*)q, q_stride_b, q_stride_h, (const T*)kmin,
                           (const T*)kmax, s_stride_b, s_stride_h, s_stride_page, alibi_slopes,
                           (T*)scores, H, Hkv, num_pages, page_size, seq_len, q_pos, seq_lens,
                           rev, nt);
        return check_launch("criticality_kernel");
      });
    });
  });
}
}  // namespace topk
}  // namespace ekv

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
      int cap = 0, list_words = 0;
      const int64_t sel_lds = select_lds_bytes(G, num_pages, k, &cap, &list_words);
      EKV_REQUIRE(sel_lds >= 0, "ekv_topk_pages: group top-k of %d of %d pages does not fit LDS",
                  k, num_pages);
      auto kern = topk_kernel<T, G>;
      if (int rc = set_lds((const void*)kern, sel_lds, "topk_kernel")) return rc;
      hipLaunchKernelGGL(kern, dim3(B * Hkv), dim3(kThreads), (size_t)sel_lds, s,
                         (const T*)scores, H, Hkv, num_pages, k, last_page, 1, nullptr,
                         page_indices, pi_stride_b, pi_stride_h, cap, list_words);
      return check_launch("topk_kernel");
    });
  });
}
