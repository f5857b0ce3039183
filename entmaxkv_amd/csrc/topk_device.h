// Device-side building blocks of page criticality and top-k page selection
// (kernels/page_criticality.py:24-104, attention_topk.py:52-71), shared by the
// criticality launches and the fused top-k decode launch.
#pragma once

#include <atomic>

#include "ekv_common.h"

// Phase timestamps (experiment builds define EKV_CSTAMP before including).
#ifndef EKV_CSTAMP
#define EKV_CSTAMP(i)
#endif
#ifndef EKV_WSTAMP
#define EKV_WSTAMP(i)
#endif
#ifndef EKV_SSTAMP
#define EKV_SSTAMP(i)
#endif

namespace ekv {
namespace topk {


constexpr int kThreads = 256;
constexpr int kUnroll = 4;  // pages per segment per workgroup
// Page keys staged in LDS by the top-k pass (16384 pages = 256k tokens at
// page size 16, 64 KB); longer caches re-read the scores on every pass.
constexpr int kMaxStagedKeys = 16384;
// Static LDS the top-k kernels of criticality_topk.hip may use (their group
// histograms; 37 KB at fp32 and G = 8): the dynamic LDS sizing leaves it free.
constexpr int kSelectStaticLds = 40960;

// Consecutive criticality scans read the bounds in opposite orders (returns 0
// or 1 alternately, over the whole process), so that a step starts with the
// pages the last one read most recently: the GPU's memory-side cache (256 MB)
// holds the tail of the last step's 268 MB at the headline shape, and an
// unchanged order would evict each line just before it is read again.  Every
// result is the same in either order (each page's score and key is computed
// alone; the key histogram is an integer count).  A launch captured in a
// graph keeps the order of its capture.
inline int next_scan_order() {
  static std::atomic<unsigned> scans{0};
  return (int)(scans.fetch_add(1, std::memory_order_relaxed) & 1u);
}

// Host launcher (criticality_topk.hip) of the criticality scores alone over
// many workgroups per (b, kv head), whatever the head count: the fused top-k
// step runs it first when one workgroup per head would leave CUs idle.  `rev`
// reverses the order in which its workgroups take their pages; `nt` makes its
// loads non-temporal (kStreamNtBytes).
int criticality_split_scores(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                             const void* kmin, const void* kmax, int64_t s_stride_b,
                             int64_t s_stride_h, int64_t s_stride_page,
                             const float* alibi_slopes, void* scores, int B, int H, int Hkv,
                             int D, int num_pages, int page_size, int seq_len, int q_pos,
                             const int32_t* seq_lens, int dtype, hipStream_t s, int rev = 0,
                             int nt = 0);

// Top-k geometry of batch element b.  With per-sequence lengths, sequence b
// scores its pages [0, P_b - 1) (the partial last page excluded), selects
// min(k, P_b - 1) of them and, when the caller asks for the sentinel
// (last_page >= 0), appends its own last page P_b - 1 (attention_topk.py:
// 49-71 per sequence); seq_len / q_pos of the ALiBi bonus are its own.
// Without lengths, the uniform values.  `stride` is the score row stride
// (the longest sequence's scored pages).
struct Ragged {
  int count, k, last_page, seq_len, q_pos;
};
__device__ __forceinline__ Ragged ragged_topk(const int32_t* seq_lens, int b, int ps, int stride,
                                              int seq_len, int q_pos, int k, int last_page) {
  Ragged r;
  if (!seq_lens) {
    r.count = stride;
    r.k = k;
    r.last_page = last_page;
    r.seq_len = seq_len;
    r.q_pos = q_pos;
    return r;
  }
  const int len = seq_lens[b];
  const int pages = (len + ps - 1) / ps;
  r.count = min(max(pages - 1, 0), stride);
  r.k = k < 0 ? k : min(k, r.count);
  r.last_page = last_page < 0 ? last_page : pages - 1;
  r.seq_len = len;
  r.q_pos = len - 1;
  return r;
}

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

// Adds one to hist[bin] for every active lane of the wave; lanes that share a
// bin add together with one LDS atomic (the top digit of the page scores falls
// into a handful of bins, and same-address atomics serialise).  The loop runs
// once per distinct bin among the active lanes.
__device__ __forceinline__ void wave_hist_add(unsigned* hist, uint32_t bin, bool act) {
  uint64_t m = __ballot(act);
  while (m) {
    const int leader = (int)__builtin_ctzll(m);
    const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)bin, leader);
    const uint64_t same = __ballot(act && bin == b);
    if ((int)(threadIdx.x & 63) == leader) atomicAdd(&hist[b], (unsigned)__popcll(same));
    m &= ~same;
    if (bin == b) act = false;
  }
}

// Radix select over the keys key_of(p), p in [0, n), for 0 < k < n: `thr`
// is the k-th largest key and `kk` how many keys equal to it are taken (the
// first ones in page order).  8 bits per pass from the top, kBits / 8 passes:
// one histogram per pass (LDS atomics), then every wave scans the 256 bins
// itself (DPP prefix sum + ballot) to find the bin of the k-th largest key, so
// a pass costs one barrier.  `hist` must be zero and visible to every thread
// on entry.  Pass 0 adds through wave_hist_add (one atomic per distinct bin
// per wave); later passes too when kAggregate (keys with many duplicates,
// whose plain atomics would serialise on a few addresses).
template <int NT, int kBits, typename KeyOf, bool kAggregate = false>
__device__ __forceinline__ void radix_threshold(KeyOf key_of, int n, int k,
                                                unsigned (*hist)[256], uint32_t& thr,
                                                int& kk, const unsigned* pass0 = nullptr) {
  constexpr int kPasses = kBits / 8;
  constexpr int kBatch = 8;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  uint32_t prefix = 0, pmask = 0;
  kk = k;
#pragma unroll
  for (int pass = 0; pass < kPasses; ++pass) {
    const int shift = kBits - 8 * (pass + 1);
    // pass 0 may come prebuilt (the criticality scan adds every key's top
    // digit as it goes) and already visible to every thread
    const bool prebuilt = pass == 0 && pass0 != nullptr;
    const unsigned* hp = prebuilt ? pass0 : hist[pass];
    if (!prebuilt) {
      for (int p0 = 0; p0 < n; p0 += NT * kBatch) {
        uint32_t kv[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int p = p0 + j * NT + tid;
          kv[j] = p < n ? key_of(p) : 0u;
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int p = p0 + j * NT + tid;
          const bool act = p < n && (kv[j] & pmask) == prefix;
          const uint32_t bin = (kv[j] >> shift) & 255u;
          if (pass == 0 || kAggregate) {
            // wave-uniform: every lane takes part in the ballots
            if (p0 + j * NT < n) wave_hist_add(hist[pass], bin, act);
          } else if (act) {
            atomicAdd(&hist[pass][bin], 1u);
          }
        }
      }
      EKV_WSTAMP(1 + pass);
      __syncthreads();
    }
    // lane l holds bins 255-4l .. 252-4l; the bin where the count from the
    // top reaches kk is found by every wave independently
    const int top = 255 - 4 * lane;
    const int c0 = (int)hp[top], c1 = (int)hp[top - 1];
    const int c2 = (int)hp[top - 2], c3 = (int)hp[top - 3];
    const int sum = c0 + c1 + c2 + c3;
    const int incl = wave_incl_scan(sum);
    const int excl = incl - sum;
    const uint64_t hit = __ballot(excl < kk && incl >= kk);
    const int src = (int)__builtin_ctzll(hit);  // at least kk keys share the prefix
    int e = excl, bin, rem;
    if (e + c0 >= kk) {
      bin = top;
      rem = kk - e;
    } else if ((e += c0) + c1 >= kk) {
      bin = top - 1;
      rem = kk - e;
    } else if ((e += c1) + c2 >= kk) {
      bin = top - 2;
      rem = kk - e;
    } else {
      e += c2;
      bin = top - 3;
      rem = kk - e;
    }
    bin = __builtin_amdgcn_readlane(bin, src);
    rem = __builtin_amdgcn_readlane(rem, src);
    prefix |= ((uint32_t)bin) << shift;
    pmask |= 255u << shift;
    kk = rem;
  }
  thr = prefix;
}

// Emits the selected pages in ascending page order, emit(slot, p, key): every
// page when `take_all`, else the keys above `thr` and the first `kk` equal to
// it.  Each wave owns a contiguous range of pages; slots come from ballots and
// the per-wave counts (`wave_cnt`, 2 * NT / 64 ints; one barrier).
template <int NT, typename KeyOf, typename Emit>
__device__ __forceinline__ void pack_selected(KeyOf key_of, int n, bool take_all, uint32_t thr,
                                              int kk, int* wave_cnt, Emit emit) {
  constexpr int W = NT / 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int per = (n + W - 1) / W;
  const int pw0 = min(n, wid * per), pw1 = min(n, pw0 + per);
  auto flags = [&](int p, bool& gt, bool& eq, uint32_t& key) {
    gt = eq = false;
    key = 0;
    if (p < pw1) {
      key = key_of(p);
      if (take_all) {
        gt = true;
      } else {
        gt = key > thr;
        eq = key == thr;
      }
    }
  };
  int gt_n = 0, eq_n = 0;
  for (int r0 = pw0; r0 < pw1; r0 += 64) {
    bool gt, eq;
    uint32_t key;
    flags(r0 + lane, gt, eq, key);
    gt_n += __popcll(__ballot(gt));
    eq_n += __popcll(__ballot(eq));
  }
  if (lane == 0) {
    wave_cnt[2 * wid] = gt_n;
    wave_cnt[2 * wid + 1] = eq_n;
  }
  EKV_WSTAMP(3);
  __syncthreads();
  EKV_CSTAMP(14);
  int gt_base = 0, eq_base = 0;
  for (int w = 0; w < wid; ++w) {
    gt_base += wave_cnt[2 * w];
    eq_base += wave_cnt[2 * w + 1];
  }
  for (int r0 = pw0; r0 < pw1; r0 += 64) {
    const int p = r0 + lane;
    bool gt, eq;
    uint32_t key;
    flags(p, gt, eq, key);
    const uint64_t mg = __ballot(gt), me = __ballot(eq);
    const int gt_rank = gt_base + __popcll(mg & below);
    const int eq_rank = eq_base + __popcll(me & below);
    if (gt || (eq && eq_rank < kk)) emit(gt_rank + min(eq_rank, kk), p, key);
    gt_base += __popcll(mg);
    eq_base += __popcll(me);
  }
}

// Radix select of G key sets at once (query head g's keys key_of(g, p)): the
// k-th largest key of each (thr[g]) and how many keys equal to it to take
// (kk[g]).  One histogram per head per pass (hist[pass][g], zero and visible
// on entry), one barrier per pass; every wave scans the G histograms itself.
template <int NT, int kBits, int G, typename KeyOf>
__device__ __forceinline__ void radix_threshold_group(KeyOf key_of, int n, int k,
                                                      unsigned (*hist)[G][256],
                                                      uint32_t (&thr)[G], int (&kk)[G]) {
  constexpr int kPasses = kBits / 8;
  constexpr int kBatch = 4;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  uint32_t prefix[G];
  uint32_t pmask = 0;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    prefix[g] = 0;
    kk[g] = k;
  }
#pragma unroll
  for (int pass = 0; pass < kPasses; ++pass) {
    const int shift = kBits - 8 * (pass + 1);
    for (int p0 = 0; p0 < n; p0 += NT * kBatch) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        uint32_t kv[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int p = p0 + j * NT + tid;
          kv[j] = p < n ? key_of(g, p) : 0u;
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int p = p0 + j * NT + tid;
          const bool act = p < n && (kv[j] & pmask) == prefix[g];
          const uint32_t bin = (kv[j] >> shift) & 255u;
          if (pass == 0) {
            if (p0 + j * NT < n) wave_hist_add(hist[pass][g], bin, act);
          } else if (act) {
            atomicAdd(&hist[pass][g][bin], 1u);
          }
        }
      }
    }
    EKV_SSTAMP(7 + 2 * pass);
    __syncthreads();
    const int top = 255 - 4 * lane;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const unsigned* h = hist[pass][g];
      const int c0 = (int)h[top], c1 = (int)h[top - 1];
      const int c2 = (int)h[top - 2], c3 = (int)h[top - 3];
      const int sum = c0 + c1 + c2 + c3;
      const int incl = wave_incl_scan(sum);
      const int excl = incl - sum;
      const uint64_t hit = __ballot(excl < kk[g] && incl >= kk[g]);
      const int src = (int)__builtin_ctzll(hit);
      int e = excl, bin, rem;
      if (e + c0 >= kk[g]) {
        bin = top;
        rem = kk[g] - e;
      } else if ((e += c0) + c1 >= kk[g]) {
        bin = top - 1;
        rem = kk[g] - e;
      } else if ((e += c1) + c2 >= kk[g]) {
        bin = top - 2;
        rem = kk[g] - e;
      } else {
        e += c2;
        bin = top - 3;
        rem = kk[g] - e;
      }
      bin = __builtin_amdgcn_readlane(bin, src);
      rem = __builtin_amdgcn_readlane(rem, src);
      prefix[g] |= ((uint32_t)bin) << shift;
      kk[g] = rem;
    }
    EKV_SSTAMP(8 + 2 * pass);
    pmask |= 255u << shift;
  }
#pragma unroll
  for (int g = 0; g < G; ++g) thr[g] = prefix[g];
}

// pack_selected for G key sets at once: emit(g, slot, p, key) for the pages
// each head selects, ascending per head.  `wave_cnt` holds 2 * G * NT / 64
// ints; one barrier.
template <int NT, int G, typename KeyOf, typename Emit>
__device__ __forceinline__ void pack_selected_group(KeyOf key_of, int n,
                                                    const uint32_t (&thr)[G],
                                                    const int (&kk)[G], int* wave_cnt,
                                                    Emit emit) {
  constexpr int W = NT / 64;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int per = (n + W - 1) / W;
  const int pw0 = min(n, wid * per), pw1 = min(n, pw0 + per);
  int gt_n[G], eq_n[G];
#pragma unroll
  for (int g = 0; g < G; ++g) gt_n[g] = eq_n[g] = 0;
  for (int r0 = pw0; r0 < pw1; r0 += 64) {
    const int p = r0 + lane;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint32_t key = p < pw1 ? key_of(g, p) : 0u;
      gt_n[g] += __popcll(__ballot(p < pw1 && key > thr[g]));
      eq_n[g] += __popcll(__ballot(p < pw1 && key == thr[g]));
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      wave_cnt[(g * W + wid) * 2] = gt_n[g];
      wave_cnt[(g * W + wid) * 2 + 1] = eq_n[g];
    }
  }
  __syncthreads();
  int gt_base[G], eq_base[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    gt_base[g] = eq_base[g] = 0;
    for (int w = 0; w < wid; ++w) {
      gt_base[g] += wave_cnt[(g * W + w) * 2];
      eq_base[g] += wave_cnt[(g * W + w) * 2 + 1];
    }
  }
  for (int r0 = pw0; r0 < pw1; r0 += 64) {
    const int p = r0 + lane;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const uint32_t key = p < pw1 ? key_of(g, p) : 0u;
      const bool gt = p < pw1 && key > thr[g];
      const bool eq = p < pw1 && key == thr[g];
      const uint64_t mg = __ballot(gt), me = __ballot(eq);
      const int gt_rank = gt_base[g] + __popcll(mg & below);
      const int eq_rank = eq_base[g] + __popcll(me & below);
      if (gt || (eq && eq_rank < kk[g])) emit(g, gt_rank + min(eq_rank, kk[g]), p, key);
      gt_base[g] += __popcll(mg);
      eq_base[g] += __popcll(me);
    }
  }
}

// Pages the sorted group select handles (a multiple of its workgroup size).
constexpr int kGroupSortedPages = 4096;

template <int G>
__device__ __forceinline__ int total_of(const int (&t)[G], int g) {
  int r = 0;
#pragma unroll
  for (int i = 0; i < G; ++i) r = i == g ? t[i] : r;
  return r;
}

__host__ __device__ constexpr int next_pow2_int(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

// The group top-k of topk_select_block for 16-bit keys, given each head's
// radix threshold thr[g] (its k-th largest key): every head's keys >= thr[g]
// go to its segment of `cand` (C2 words, G * C2 <= NT; `cnt` holds G * NT / 64
// ints) as
// (key << 16) | (0xffff - page); a candidate's rank is the number of its
// head's candidates with a larger composite (key descending, ties to the
// lower page), so ranks below k are the head's top-k; `level` (num_pages
// words) takes each page's best (rank * G + head) by atomicMin, `lvl` (k words) counts the pages whose best
// rank is r, and the smallest r* with at least k pages of rank <= r* gives
// the final selection: every page of level < r* and the lowest-numbered
// pages of level r*, packed in ascending page order by pack_selected.
template <int NT, int G, typename KeyGP, typename Emit>
__device__ __forceinline__ void group_select_sorted(KeyGP key_gp, int num_pages, int k,
                                                    const uint32_t (&thr)[G], int C2,
                                                    uint32_t* cand, uint32_t* level,
                                                    unsigned* lvl, int* cnt, int* wave_cnt,
                                                    Emit emit) {
  constexpr int W = NT / 64;
  constexpr int IT = kGroupSortedPages / NT;  // pages per thread
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  // candidate flags of this thread's pages (page p0 * NT + tid), all keys
  // read before any use; per-wave counts, then one barrier for the offsets
  uint32_t key[IT][G];
  uint64_t m[IT][G];
  int wc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) wc[g] = 0;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int p = it * NT + tid;
#pragma unroll
    for (int g = 0; g < G; ++g) key[it][g] = p < num_pages ? key_gp(g, p) : 0u;
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int p = it * NT + tid;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[it][g] = __ballot(p < num_pages && key[it][g] >= thr[g]);
      wc[g] += __popcll(m[it][g]);
    }
  }
  __syncthreads();  // the threshold histograms (lvl aliases them) are read
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) cnt[g * W + wid] = wc[g];
  }
  for (int p = tid; p < num_pages; p += NT) level[p] = 0xffffffffu;
  for (int i = tid; i < k; i += NT) lvl[i] = 0u;
  __syncthreads();
  int total[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    int base = 0, tot = 0;
    for (int w = 0; w < W; ++w) {
      const int c = cnt[g * W + w];
      base += w < wid ? c : 0;
      tot += c;
    }
    total[g] = tot;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int p = it * NT + tid;
      if ((m[it][g] >> lane) & 1ull)
        cand[g * C2 + base + __popcll(m[it][g] & below)] = (key[it][g] << 16) | (0xffffu - (uint32_t)p);
      base += __popcll(m[it][g]);
    }
    // zero padding up to a multiple of 4 for the four-wide reads below
    if (tid < 3 && tot + tid < C2) cand[g * C2 + tot + tid] = 0u;
  }
  __syncthreads();
  EKV_CSTAMP(13);
  // rank of a candidate within its head: how many of the head's candidates
  // order before it (larger composite; the padding never does); one
  // candidate per thread (G * C2 <= NT), eight four-wide LDS reads in flight
  const int e = tid;
  const int g = e / C2, slot = e % C2;
  uint32_t c = 0, rank = 0;
  if (e < G * C2 && slot < total_of(total, g)) {
    const uint32_t* seg = cand + g * C2;
    c = seg[slot];
    const uint4* s4 = reinterpret_cast<const uint4*>(seg);
    const int n4 = (total_of(total, g) + 3) / 4;
#pragma unroll 8
    for (int j = 0; j < n4; ++j) {
      const uint4 x = s4[j];
      rank += (x.x > c) + (x.y > c) + (x.z > c) + (x.w > c);
    }
    if ((int)rank < k) atomicMin(&level[0xffffu - (c & 0xffffu)], rank * (uint32_t)G + (uint32_t)g);
  }
  __syncthreads();
  EKV_CSTAMP(15);
  // each page counted once, by its best (rank, head) entry
  if (c != 0u && (int)rank < k &&
      level[0xffffu - (c & 0xffffu)] == rank * (uint32_t)G + (uint32_t)g)
    atomicAdd(&lvl[rank], 1u);
  __syncthreads();
  // r*: the smallest rank whose running page count reaches k (every wave
  // finds it itself: no barrier)
  int run = 0, rstar = k - 1, need = 0;
  for (int r0 = 0; r0 < k; r0 += 64) {
    const int r = r0 + lane;
    const int c = r < k ? (int)lvl[r] : 0;
    const int incl = run + wave_incl_scan(c);
    const uint64_t hit = __ballot(r < k && incl >= k);
    if (hit) {
      const int src = (int)__builtin_ctzll(hit);
      rstar = r0 + src;
      need = k - (__shfl(incl, src) - __shfl(c, src));
      break;
    }
    run = __shfl(incl, 63);
  }
  const uint32_t thr1 = (uint32_t)(k - rstar);
  auto key_l = [&](int p) -> uint32_t {
    const uint32_t v = level[p];
    return v == 0xffffffffu ? 0u : (uint32_t)k - v / (uint32_t)G;
  };
  pack_selected<NT>(key_l, num_pages, false, thr1, need, wave_cnt, emit);
}

// LDS words of the candidate lists (page, key, rank) of a group of G > 1
// query heads: all G lists at once (`concurrent`), else one list at a time.
__host__ __device__ constexpr int group_list_words(int G, int k, bool concurrent = true) {
  return G > 1 ? 3 * k * (concurrent ? G : 1) : 0;
}

// Block-wide top-k of one (b, kv head) over `num_pages` pages; writes
// ascending page ids to out[0..k) (and lds_out[0..k) when non-null) and
// `last_page` to out[k] when last_page >= 0.  blockDim == NT.
//
// `out` may be null: the table then goes to lds_out only (the caller stores
// it later, so that no barrier waits on the global stores).
//
// G == 1: the head's own order keys.  They come from `lds_keys` when
// `prestaged`, are staged there first when they fit (`lds_cap` keys), and are
// otherwise recomputed from the scores on every pass (the scores must be
// visible to this workgroup: written by a previous launch or by this
// workgroup).  `ext_hist` (kBits / 8 histograms of 256 bins, zero and visible
// on entry) replaces the select's own histograms; with `pass0_built` its
// first histogram already counts every key's top 8 bits (the criticality
// scan built it), which saves a pass and a barrier.
//
// G > 1 (the group shares one page table; no reference counterpart): pages
// are taken by their best rank over the group's query heads, ties to the lower
// page index -- round robin over the heads' own top-k lists.  Radix selects
// give each head's top-k list (page, key) in `lds_list` -- all G heads in the
// same passes when `list_words` >= group_list_words(G, k), else one head
// after another -- each entry's rank within its list is counted (a list is
// ascending in page order, so equal keys rank by page; every thread counts a
// slice of one list for one entry), and `lds_keys` (num_pages words,
// required: lds_cap >= num_pages) keeps each page's minimum rank.  Ranks
// become keys k - rank and one more select takes the k best.  A head's keys
// come from `head_keys[g * hk_stride + p]` when non-null, else from the
// scores.
template <typename T, int G, int NT = kThreads>
__device__ __forceinline__ void topk_select_block(const T* __restrict__ s0, int64_t head_stride,
                                                  int num_pages, int k, int last_page,
                                                  int32_t* __restrict__ out, uint32_t* lds_keys,
                                                  int lds_cap, bool prestaged = false,
                                                  int* lds_out = nullptr,
                                                  uint32_t* lds_list = nullptr,
                                                  const uint32_t* head_keys = nullptr,
                                                  int hk_stride = 0, int list_words = 0,
                                                  unsigned (*ext_hist)[256] = nullptr,
                                                  bool pass0_built = false) {
  constexpr int W = NT / 64;
  constexpr int kBits = ScoreKey<T>::kBits;
  constexpr int kPasses = kBits / 8;
  constexpr int kBatch = 8;
  __shared__ unsigned hist[kPasses][256];
  __shared__ int wave_cnt[2 * W];
  const int tid = threadIdx.x;
  k = min(k, num_pages);
  const bool take_all = (k == num_pages);
  auto emit_out = [&](int slot, int p, uint32_t) {
    if (out) out[slot] = p;
    if (lds_out) lds_out[slot] = p;
  };
  auto zero_hist = [&]() {
    for (int i = tid; i < kPasses * 256; i += NT) (&hist[0][0])[i] = 0u;
  };
  if constexpr (G == 1) {
    const bool staged = prestaged || num_pages <= lds_cap;
    auto own = [&](int p) -> uint32_t { return ScoreKey<T>::key(s0[p]); };
    auto key_of = [&](int p) -> uint32_t { return staged ? lds_keys[p] : own(p); };
    unsigned (*hs)[256] = ext_hist ? ext_hist : hist;
    if (!ext_hist) zero_hist();
    if (staged && !prestaged) {
      for (int p0 = 0; p0 < num_pages; p0 += NT * kBatch) {
        uint32_t kv[kBatch];
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int p = p0 + j * NT + tid;
          kv[j] = p < num_pages ? own(p) : 0u;
        }
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int p = p0 + j * NT + tid;
          if (p < num_pages) lds_keys[p] = kv[j];
        }
      }
    }
    if (!ext_hist || (staged && !prestaged)) __syncthreads();
    EKV_CSTAMP(2);
    uint32_t thr = 0;
    int kk = 0;
    if (k > 0 && !take_all)
      radix_threshold<NT, kBits>(key_of, num_pages, k, hs, thr, kk,
                                 ext_hist && pass0_built ? ext_hist[0] : nullptr);
    EKV_CSTAMP(3);
    if (k > 0) pack_selected<NT>(key_of, num_pages, take_all, thr, kk, wave_cnt, emit_out);
  } else {
    uint32_t* level = lds_keys;
    // the final select runs on keys k - rank <= k <= 16384: one 8-bit pass
    // when k < 256, else two; most pages share key 0, so every pass
    // aggregates its adds
    auto select_levels = [&](auto key_l, uint32_t& thr, int& kk) {
      if (k < 256)
        radix_threshold<NT, 8, decltype(key_l), true>(key_l, num_pages, k, hist, thr, kk);
      else
        radix_threshold<NT, 16, decltype(key_l), true>(key_l, num_pages, k, hist, thr, kk);
    };
    auto key_gp = [&](int g, int p) -> uint32_t {
      return head_keys ? head_keys[g * hk_stride + p]
                       : ScoreKey<T>::key(s0[g * head_stride + p]);
    };
    if (k > 0 && !take_all && list_words >= group_list_words(G, k)) {
      __shared__ unsigned ghist[kPasses][G][256];
      __shared__ int gwave_cnt[2 * G * W];
      uint32_t* list_page = lds_list;              // [G][k]
      uint32_t* list_key = lds_list + G * k;       // [G][k]
      uint32_t* list_rank = lds_list + 2 * G * k;  // [G][k]
      for (int p = tid; p < num_pages; p += NT) level[p] = (uint32_t)k;
      for (int i = tid; i < kPasses * G * 256; i += NT) (&ghist[0][0][0])[i] = 0u;
      for (int i = tid; i < G * k; i += NT) list_rank[i] = 0u;
      __syncthreads();
      uint32_t thr[G];
      int kk[G];
      radix_threshold_group<NT, kBits, G>(key_gp, num_pages, k, ghist, thr, kk);
      EKV_CSTAMP(12);
      // 16-bit keys: each head's candidates (keys >= its threshold) are
      // sorted in LDS instead of packed in page order and ranked pairwise,
      // and the levels are counted instead of radix-selected
      if constexpr (kBits == 16 && NT >= 1024) {
        const int c1 = next_pow2_int(k);
        const int C2 = (2 * c1 <= 3 * k) ? 2 * c1 : c1;
        int cmax = 0;
#pragma unroll
        for (int g = 0; g < G; ++g)
          cmax = max(cmax, k - kk[g] + (int)ghist[kPasses - 1][g][thr[g] & 255u]);
        if (cmax <= C2 && G * C2 <= list_words && G * C2 <= NT && k <= kPasses * G * 256 &&
            num_pages <= kGroupSortedPages && C2 >= 4) {
          group_select_sorted<NT, G>(key_gp, num_pages, k, thr, C2, lds_list, level,
                                     &ghist[0][0][0], gwave_cnt, wave_cnt, emit_out);
          if (tid == 0 && last_page >= 0) {
            if (out) out[k] = last_page;
            if (lds_out) lds_out[k] = last_page;
          }
          EKV_CSTAMP(4);
          return;
        }
      }
      pack_selected_group<NT, G>(key_gp, num_pages, thr, kk, gwave_cnt,
                                 [&](int g, int slot, int p, uint32_t key) {
                                   list_page[g * k + slot] = (uint32_t)p;
                                   list_key[g * k + slot] = key;
                                 });
      __syncthreads();
      EKV_CSTAMP(13);
      // work item w: entry i of list g against slice s of that list
      const int entries = G * k;
      const int slices = entries < NT ? NT / entries : 1;
      const int per = (k + slices - 1) / slices;
      for (int w = tid; w < entries * slices; w += NT) {
        const int e = w % entries, g = e / k, i = e % k;
        const int j0 = (w / entries) * per, j1 = min(k, j0 + per);
        const uint32_t* lk = list_key + g * k;
        const uint32_t ki = lk[i];
        uint32_t cnt = 0;
        for (int j = j0; j < j1; ++j) {
          const uint32_t kj = lk[j];
          cnt += (kj > ki) | ((kj == ki) & (j < i));
        }
        if (cnt) atomicAdd(&list_rank[e], cnt);
      }
      __syncthreads();
      for (int e = tid; e < entries; e += NT) atomicMin(&level[list_page[e]], list_rank[e]);
      __syncthreads();
      EKV_CSTAMP(14);
      for (int p = tid; p < num_pages; p += NT) level[p] = (uint32_t)k - level[p];
      zero_hist();
      __syncthreads();
      auto key_l = [&](int p) -> uint32_t { return level[p]; };
      uint32_t thr1;
      int kk1;
      select_levels(key_l, thr1, kk1);
      EKV_CSTAMP(15);
      pack_selected<NT>(key_l, num_pages, false, thr1, kk1, wave_cnt, emit_out);
    } else if (k > 0 && !take_all) {
      for (int p = tid; p < num_pages; p += NT) level[p] = (uint32_t)k;
      uint32_t* list_page = lds_list;
      uint32_t* list_key = lds_list + k;
      uint32_t* list_rank = lds_list + 2 * k;
      const int slices = k < NT ? NT / k : 1;
      const int per = (k + slices - 1) / slices;
#pragma unroll 1
      for (int g = 0; g < G; ++g) {
        auto key_g = [&](int p) -> uint32_t { return key_gp(g, p); };
        // the barrier also ends the previous head's use of the list
        zero_hist();
        for (int i = tid; i < k; i += NT) list_rank[i] = 0u;
        __syncthreads();
        uint32_t thr;
        int kk;
        radix_threshold<NT, kBits>(key_g, num_pages, k, hist, thr, kk);
        pack_selected<NT>(key_g, num_pages, false, thr, kk, wave_cnt,
                          [&](int slot, int p, uint32_t key) {
                            list_page[slot] = (uint32_t)p;
                            list_key[slot] = key;
                          });
        __syncthreads();
        // thread t counts list entries [s * per, s * per + per) against
        // entry t % k (slice s = t / k); the lanes of a wave read the same
        // key at a time (LDS broadcast)
        for (int w = tid; w < k * slices; w += NT) {
          const int i = w % k, j0 = (w / k) * per, j1 = min(k, j0 + per);
          const uint32_t ki = list_key[i];
          uint32_t cnt = 0;
          for (int j = j0; j < j1; ++j) {
            const uint32_t kj = list_key[j];
            cnt += (kj > ki) | ((kj == ki) & (j < i));
          }
          if (cnt) atomicAdd(&list_rank[i], cnt);
        }
        __syncthreads();
        for (int i = tid; i < k; i += NT) atomicMin(&level[list_page[i]], list_rank[i]);
      }
      __syncthreads();
      for (int p = tid; p < num_pages; p += NT) level[p] = (uint32_t)k - level[p];
      zero_hist();
      __syncthreads();
      auto key_l = [&](int p) -> uint32_t { return level[p]; };
      uint32_t thr;
      int kk;
      select_levels(key_l, thr, kk);
      pack_selected<NT>(key_l, num_pages, false, thr, kk, wave_cnt, emit_out);
    } else if (k > 0) {
      pack_selected<NT>([](int) -> uint32_t { return 0u; }, num_pages, true, 0u, 0, wave_cnt,
                        emit_out);
    }
  }
  if (tid == 0 && last_page >= 0) {
    if (out) out[k] = last_page;
    if (lds_out) lds_out[k] = last_page;
  }
  EKV_CSTAMP(4);
}

// Agent-scope (write-through) store and load of one storage element: a store
// reaches the level every XCD reads before the wave's waitcnt returns, and a
// load is served from there, so two workgroups on different XCDs can hand
// data over without a fence (see the paired top-k launch).
template <typename T>
__device__ __forceinline__ void store_through(T* p, T v) {
  if constexpr (sizeof(T) == 4) {
    __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(uint32_t, v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    __hip_atomic_store(reinterpret_cast<uint16_t*>(p), __builtin_bit_cast(uint16_t, v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
template <typename T>
__device__ __forceinline__ T load_through(const T* p) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __hip_atomic_load(reinterpret_cast<const uint32_t*>(p),
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  } else {
    return __builtin_bit_cast(T, __hip_atomic_load(reinterpret_cast<const uint16_t*>(p),
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  }
}

// Criticality scan of one (b, kv head) by a workgroup of NT threads: scores
// of the G query heads for pages [0, count) written to `scores`
// ([B, H, stride], query dtype; count <= stride) and, when `lds_keys` is
// non-null, the order keys kept there: lds_keys[p] for G == 1, lds_keys[g *
// stride + p] per query head for G > 1; for G == 1 with `hist0` (256 bins,
// zero and visible on entry) every key's top 8 bits are counted there too.  A
// row segment of LPR lanes owns one page and loads its min and max rows with
// 16-byte loads, U pages per segment in flight.  Returns the head's score
// base pointer.  Chunked, the scan covers pages [p_begin, num_pages) only,
// and kThrough stores the scores with store_through.
template <typename T, int LPR, int G, int NT, int U, bool kChunked = false,
          bool kThrough = false>
__device__ __forceinline__ T* criticality_scan_head(
    const T* __restrict__ q, int64_t qsb, int64_t qsh, const T* __restrict__ kmin,
    const T* __restrict__ kmax, int64_t ssb, int64_t ssh, int64_t ssp,
    const float* __restrict__ slopes, T* __restrict__ scores, int H, int stride, int num_pages,
    int page_size, int seq_len, int q_pos, int b, int kvh, uint32_t* lds_keys,
    unsigned* hist0 = nullptr, int* lds_next = nullptr, bool rev = false, bool nt = false,
    int p_begin = 0) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SEGS = NT / LPR;
  constexpr int ROUND = SEGS * U;
  const int seg = threadIdx.x / LPR;
  const int sl = threadIdx.x % LPR;
  const int col = sl * VEC;
  const int h0 = kvh * G;
  const bool keep_keys = lds_keys != nullptr;

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
  T* sbase = scores + ((int64_t)b * H + h0) * stride;

  // pages base + u * step + off for u < U
  auto body = [&](int base, int step, int off) {
    uint4 lo[U], hi[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = base + u * step + off;
      if (p < num_pages) {
        lo[u] = ld16_sel(kmn + (int64_t)p * ssp + col, nt);
        hi[u] = ld16_sel(kmx + (int64_t)p * ssp + col, nt);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = base + u * step + off;
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
        key = ScoreKey<T>::key(sv);
        if (p < num_pages && sl == 0) {
          if constexpr (kThrough) store_through(sbase + (int64_t)g * stride + p, sv);
          else sbase[(int64_t)g * stride + p] = sv;
          if (G > 1 && keep_keys) lds_keys[g * stride + p] = key;
        }
      }
      if (G == 1 && keep_keys && p < num_pages && sl == 0) {
        lds_keys[p] = key;
        if (hist0) atomicAdd(&hist0[key >> (ScoreKey<T>::kBits - 8)], 1u);
      }
    }
  };
  if constexpr (kChunked) {
    // waves take chunks of U * (64 / LPR) consecutive pages from a shared
    // counter (zero and visible on entry), the next chunk's index fetched
    // while the current chunk's loads are in flight: a wave slowed by its
    // memory accesses takes fewer chunks, so the waves finish together
    constexpr int WSEG = 64 / LPR;
    constexpr int CHUNK = WSEG * U;
    const int lane = threadIdx.x & 63;
    auto grab = [&]() {
      int v = 0;
      if (lane == 0) v = atomicAdd(lds_next, 1);
      return __builtin_amdgcn_readfirstlane(v);
    };
    // rev: the chunks are handed out last first
    const int nch = (num_pages - p_begin + CHUNK - 1) / CHUNK;
    int c = grab();
    while (c < nch) {
      const int c_next = grab();
      body(p_begin + (rev ? nch - 1 - c : c) * CHUNK, WSEG, seg % WSEG);
      c = c_next;
    }
  } else {
    for (int p0 = 0; p0 < num_pages; p0 += ROUND) body(p0, SEGS, seg);
  }
  EKV_WSTAMP(0);
  return sbase;
}

}  // namespace topk
}  // namespace ekv
