// Definitions of the per-(T, G) host launchers declared in decode_device.h.
// Included only by decode_inst.hip, which instantiates them for one pair.
#pragma once

#include "decode_device.h"

namespace ekv {
namespace dec {

// Sets the dynamic LDS of `kern` to `bytes` (a no-op for 0).
inline int set_dynamic_lds(const void* kern, size_t bytes, const char* what) {
  if (bytes == 0) return EKV_OK;
  const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)bytes);
  if (e != hipSuccess)
    return set_error(EKV_ERR_HIP, "%s LDS %zu: %s", what, bytes, hipGetErrorString(e));
  return EKV_OK;
}

// LDS a kernel's static allocation leaves for dynamic use, or -1 on error.
inline int64_t lds_left(const void* kern, const char* what) {
  hipFuncAttributes attr;
  const hipError_t e = hipFuncGetAttributes(&attr, kern);
  if (e != hipSuccess) {
    set_error(EKV_ERR_HIP, "%s attributes: %s", what, hipGetErrorString(e));
    return -1;
  }
  return (int64_t)kLdsPerWorkgroup - (int64_t)attr.sharedSizeBytes;
}

template <typename T, int G>
int Launch<T, G>::decode(DecodeArgs a, int B, int Hkv, int D, bool head_path, hipStream_t s) {
  return dispatch_lpr<T>(D, [&](auto lpr) {
    constexpr int LPR = decltype(lpr)::value;
    constexpr int U = G >= 4 ? 2 : 8 / G;
    if (!head_path) {
      hipLaunchKernelGGL((score_split_kernel<T, LPR, G>), dim3(a.splits, B * Hkv),
                         dim3(kSplitThreads), 0, s, a);
      const int rc = check_launch("score_split_kernel");
      if (rc) return rc;
    }
    auto kern = decode_head_kernel<T, LPR, G, U>;
    if (a.stage_cap > 0) {
      const int64_t avail = lds_left((const void*)kern, "decode_head_kernel");
      if (avail < 0) return EKV_ERR_HIP;
      const int64_t fit = avail / (4 * G);
      if (fit < a.stage_cap) a.stage_cap = (int)fit;
    }
    const size_t lds = (size_t)a.stage_cap * G * sizeof(float);
    const int rc = set_dynamic_lds((const void*)kern, lds, "decode_head_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(kern, dim3(B * Hkv), dim3(kHeadThreads), lds, s, a);
    return check_launch("decode_head_kernel");
  });
}

template <typename T, int G>
int Launch<T, G>::topk(DecodeArgs a, SelectArgs t, int B, int Hkv, int D, int tokens,
                       hipStream_t s, int* handled) {
  *handled = 0;
  return dispatch_lpr<T>(D, [&](auto lpr) {
    constexpr int LPR = decltype(lpr)::value;
    // pages per row segment in flight in the criticality scan: two measured
    // faster than four for a lone group (more requests in flight per CU only
    // queue up); the G query heads of a group share every page load
    constexpr int UC = G >= 8 ? 1 : (G == 1 ? 2 : 8 / G);
    constexpr int UD = G >= 4 ? 2 : 8 / G;
    // the paired launch or the one-workgroup launch
    auto kern = t.pair_cnt ? topk_decode_kernel<T, LPR, G, UC, UD, true>
                           : topk_decode_kernel<T, LPR, G, UC, UD>;
    const int64_t avail = lds_left((const void*)kern, "topk_decode_kernel");
    if (avail < 0) return EKV_ERR_HIP;
    // keys (G == 1), or page ranks + candidate lists (all G at once when they
    // fit, else one) + every head's keys when they fit (else the selection
    // re-reads the scores) for G > 1; the decode scores reuse the same LDS
    // afterwards.  The first layout that fits wins.
    const int64_t stage = (int64_t)tokens * G * 4;
    t.head_keys = 0;
    t.list_words = 0;
    int64_t lds = -1;
    if (G == 1) {
      const int64_t sel = (int64_t)t.num_pages * 4;
      lds = sel > stage ? sel : stage;
    } else {
      for (int variant = 0; variant < 4 && lds < 0; ++variant) {
        const bool concurrent = variant == 0 || variant == 2;
        const bool keys_in_lds = variant < 2;
        const int words = topk::group_list_words(G, t.k, concurrent);
        int64_t sel = ((int64_t)t.num_pages + words) * 4;
        if (keys_in_lds) sel += (int64_t)G * t.num_pages * 4;
        const int64_t need = sel > stage ? sel : stage;
        if (need <= avail) {
          lds = need;
          t.list_words = words;
          t.head_keys = keys_in_lds ? 1 : 0;
        }
      }
    }
    if (lds < 0 || lds > avail) return EKV_OK;  // too big: the caller falls back
    // the paired launch of groups hands every query head's keys over in LDS
    if (G > 1 && t.pair_cnt && !t.head_keys) return EKV_OK;
    const int rc = set_dynamic_lds((const void*)kern, (size_t)lds, "topk_decode_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(kern, dim3(B * Hkv * (t.pair_cnt ? 2 : 1)), dim3(kHeadThreads),
                       (size_t)lds, s, a, t);
    *handled = 1;
    return check_launch("topk_decode_kernel");
  });
}

template <typename T, int G>
int Launch<T, G>::gaussian(DecodeArgs a, GaussArgs f, int B, int Hkv, int D, int max_tokens,
                           hipStream_t s) {
  return dispatch_lpr<T>(D, [&](auto lpr) {
    constexpr int LPR = decltype(lpr)::value;
    constexpr int UD = G >= 4 ? 2 : 8 / G;
    auto kern = f.pair_cnt ? gaussian_decode_kernel<T, LPR, G, UD, true>
                           : gaussian_decode_kernel<T, LPR, G, UD>;
    // scores stay in LDS up to what the static LDS leaves (else the workspace)
    const int64_t avail = lds_left((const void*)kern, "gaussian_decode_kernel");
    if (avail < 0) return EKV_ERR_HIP;
    int64_t cap = avail / (4 * G);
    if (cap > max_tokens) cap = max_tokens;
    a.stage_cap = (int)cap;
    const size_t lds = (size_t)cap * G * sizeof(float);
    const int rc = set_dynamic_lds((const void*)kern, lds, "gaussian_decode_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(kern, dim3(B * Hkv * (f.pair_cnt ? 2 : 1)), dim3(kHeadThreads), lds, s,
                       a, f);
    return check_launch("gaussian_decode_kernel");
  });
}

}  // namespace dec
}  // namespace ekv
