// Device-side building blocks of page criticality and top-k page selection
// (kernels/page_criticality.py:24-104, attention_topk.py:52-71), shared by the
// criticality launches and the fused top-k decode launch.
#pragma once

#include "ekv_common.h"

#ifdef EKV_PHASE_TIMERS
extern __device__ unsigned long long ekv_crit_timers[4096 * 8];
#define EKV_CSTAMP(i) \
  if (threadIdx.x == 0 && blockIdx.x < 4096) ekv_crit_timers[blockIdx.x * 8 + (i)] = wall_clock64()
#else
#define EKV_CSTAMP(i)
#endif

namespace ekv {
namespace topk {


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

  EKV_CSTAMP(2);
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
  EKV_CSTAMP(3);
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
  EKV_CSTAMP(4);
}

// One workgroup of kHeadThreads per (b, kv head): scores every page of the
// head (16-byte loads, kHeadUnroll pages per row segment in flight), keeps
// the group-max keys in LDS and, when k_sel >= 0, selects the top-k pages in
// the same workgroup.  No cross-workgroup communication.
constexpr int kHeadThreads = 512;
constexpr int kHeadUnroll = 8;


}  // namespace topk
}  // namespace ekv
