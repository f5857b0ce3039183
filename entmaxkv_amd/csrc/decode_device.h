// Paged alpha-entmax decode over a compacted page table.
//
// Follows kernels/adadecode_paged.py:567-762 (exact tau: global max,
// 16-bin histogram init, bracketed Halley, output) and
// kernels/adadecode_paged_gaussian_tau.py:192-331 (given tau: unbounded
// Halley/Newton corrections, output).  Compacted token c of (b, kv head) lives
// in cache row page_indices[c / ps] * ps + c % ps; scores are
// s_c = qs . k_c with qs = q * (alpha-1)/sqrt(D) rounded to the input dtype,
// and out = sum_c [s_c - tau]_+^(1/(alpha-1)) v_c (not renormalised, as in
// the reference).
//
// One workgroup of 1024 threads owns one (b, kv head) and all G query heads
// of its group, so nothing crosses workgroups:
//   phase 1  stream the selected K rows once (16-byte loads, one load serves
//            all G heads) and keep the fp32 scores in LDS (in the workspace
//            when they do not fit);
//   phase 2  solve tau per head over those scores (one wave per head, or the
//            whole workgroup per head for long token lists);
//   phase 3  compact the tokens with s > tau (the entmax support), gather only
//            those V rows and reduce in registers/LDS; write out.
// When batch * kv heads is too small to fill the GPU, phase 1 runs as a
// separate split launch over many workgroups per head (score_split_kernel)
// and the head kernel starts at phase 2.  The reference launches 7 + 2*niter
// kernels and reads K 3 + niter times.
#pragma once

// Experiment builds only (-DEKV_PHASE_TIMERS on one decode_inst unit):
// per-workgroup wall-clock stamps (100 MHz) of the fused kernels' phases.
#ifdef EKV_PHASE_TIMERS
__device__ unsigned long long ekv_phase_timers[4096 * 16];
// per-wave stamps: [block < 256][wave][slot < 8]
__device__ unsigned long long ekv_wave_timers[256 * 16 * 8];
#define EKV_WSTAMP(i)                                                    \
  if ((threadIdx.x & 63) == 0 && blockIdx.x < 256)                       \
  ekv_wave_timers[(blockIdx.x * 16 + (threadIdx.x >> 6)) * 8 + (i)] = wall_clock64()
#define EKV_STAMP(i) \
  if (threadIdx.x == 0 && blockIdx.x < 4096) ekv_phase_timers[blockIdx.x * 16 + (i)] = wall_clock64()
#ifdef EKV_SEL_STAMPS
#define EKV_TSTAMP(i)
#define EKV_SSTAMP(i) EKV_STAMP(i)
#else
#define EKV_TSTAMP(i) EKV_STAMP(i)
#define EKV_SSTAMP(i)
#endif
// slot 6 in the top-k launch: the top-k threshold found (topk_device.h stamp
// 3); slots 12-15: the group select's stages (stamps 12-15)
#define EKV_CSTAMP(i)  \
  do {                  \
    if ((i) == 3) {     \
      EKV_STAMP(6);     \
    } else if ((i) >= 12) { \
      EKV_STAMP(i);     \
    }                   \
  } while (0)
#else
#define EKV_STAMP(i)
#define EKV_WSTAMP(i)
#define EKV_TSTAMP(i)
#define EKV_SSTAMP(i)
#endif

#include "ekv_common.h"
#include "topk_device.h"
#include "gaussian_device.h"
#include "append_device.h"

namespace ekv {
namespace dec {


constexpr int kSplitThreads = 256;
constexpr int kSplitUnroll = 4;
constexpr int kSplitTablePages = 1024;  // page ids staged in LDS per chunk of a split
constexpr int kHeadThreads = 1024;
constexpr int kWaves = kHeadThreads / 64;
constexpr int kBins = 16;
constexpr int kBatch = 8;           // independent loads per lane in score passes
constexpr int kTablePages = 2048;   // page ids staged in LDS per phase-1 chunk
// tokens whose support the V phase compacts at once (two per thread for G <= 2)
__host__ __device__ constexpr int sup_chunk(int G) { return G <= 2 ? 2 * kHeadThreads : kHeadThreads; }

struct DecodeArgs {
  const void* q;
  int64_t qsb, qsh;
  const void* k;
  const void* v;
  int64_t ksb, ksh, ksr;
  int64_t row_limit;  // rows addressable in each (b, kv head) of K/V
  // Block pool (null: contiguous cache).  Row r of (b, kv head) then lives in
  // block block_table[b * btsb + r / page_size] at
  // block * ksb + kvh * ksh + (r % page_size) * ksr; ids outside [0,
  // bt_blocks) are skipped like out-of-range page ids.
  const int32_t* block_table = nullptr;
  int64_t btsb = 0;
  int bt_blocks = 0;
  const int32_t* page_indices;
  int64_t pisb, pish;
  int n_slots;
  const int32_t* cache_seqlens;
  int64_t csb, csh;
  const int32_t* q_seqlens;
  const float* slopes;
  // ALiBi key positions [B, Hkv, rows] (null: a key's position is its cache row)
  const int32_t* positions = nullptr;
  int64_t posb = 0, posh = 0;
  float* tau;           // [B, H] output
  const float* tau_in;  // [B, H] starting tau (given-tau mode)
  int tau_mode;         // 0 exact (histogram + bracketed Halley), 1 given tau (unbounded Halley)
  int iters;
  void* out;
  int64_t osb, osh;
  float alpha;
  float qscale;  // (alpha-1)/sqrt(D) already rounded to the input dtype
  int page_size;
  int H, Hkv;
  int splits;        // phase-1 workgroups per head in the split path
  int max_tokens;    // row stride of the workspace scores
  float* ws_scores;  // [B, H, max_tokens]
  int stage_cap;     // scores per head kept in LDS (0: workspace)
  int scores_ready;  // phase 1 already done by score_split_kernel
};

__device__ __forceinline__ int token_count(const DecodeArgs& a, int b, int kvh) {
  int n = a.cache_seqlens[b * a.csb + kvh * a.csh];
  n = max(n, 0);
  return min(n, min(a.n_slots * a.page_size, a.max_tokens));
}

// Maps compacted token c to its cache row, or -1 when the page id is outside
// the cache (a malformed table never causes an out-of-bounds access).
__device__ __forceinline__ int64_t token_row(const int32_t* __restrict__ pi, int c, int ps,
                                             int64_t row_limit) {
  const int page = pi[c / ps];
  const int64_t row = (int64_t)page * ps + (c % ps);
  return (page >= 0 && row < row_limit) ? row : -1;
}

__device__ __forceinline__ float entmax_weight(float x, float alpha, float c0) {
  if (alpha == 2.0f) return x;
  if (alpha == 1.5f) return x * x;
  return exp2f(log2f(x) * c0);
}

// Element offset of cache row `row` of (b, kv head) from the K/V base
// pointer, or -1 when the row lies outside the cache (contiguous rows, or a
// block of the pool; see DecodeArgs::block_table).
__device__ __forceinline__ int64_t kv_row_offset(const DecodeArgs& a, int b, int kvh,
                                                 int64_t row) {
  if (row < 0 || row >= a.row_limit) return -1;
  if (!a.block_table) return b * a.ksb + kvh * a.ksh + row * a.ksr;
  const int blk = a.block_table[b * a.btsb + row / a.page_size];
  if (blk < 0 || blk >= a.bt_blocks) return -1;
  return blk * a.ksb + kvh * a.ksh + (row % a.page_size) * a.ksr;
}

// q * qscale rounded to the storage dtype, kept in the storage format
// (kernels/adadecode_paged.py:97-98).
template <typename T, int G>
__device__ __forceinline__ void load_query(const DecodeArgs& a, int b, int h0, int col,
                                           uint4 (&qraw)[G]) {
  constexpr int VEC = 16 / sizeof(T);
  const T* qb = (const T*)a.q + b * a.qsb;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    Vec<T> x;
    x.load(qb + (h0 + g) * a.qsh + col);
#pragma unroll
    for (int i = 0; i < VEC; ++i) x.v[i] = x.v[i] * a.qscale;
    T tmp[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) tmp[i] = from_f<T>(x.v[i]);
    qraw[g] = *reinterpret_cast<const uint4*>(tmp);
  }
}

// ---------------------------------------------------------------------------
// GQA scoring on the matrix cores
// ---------------------------------------------------------------------------
//
// With G query heads per kv head the scores of 16 tokens are a 16 x D by
// D x G product.  v_mfma_f32_16x16x32_{f16,bf16} computes a 16 x 16 tile of
// it per 32-wide slice of D (G of the 16 columns used), in place of G dot
// products and G 16-lane reductions per token on the VALU, which bound the
// scoring phase for G >= 2.  Operand layout (lane l, measured on gfx950):
// A[l % 16][8 (l / 16) + e] (e < 8), B[8 (l / 16) + e][l % 16], and the
// result C[4 (l / 16) + r][l % 16] (r < 4).  Products of 16-bit values are
// exact in fp32 and the accumulation is fp32, as on the VALU path; only the
// summation order differs.
#ifndef EKV_MFMA_MIN_G
#define EKV_MFMA_MIN_G 2
#endif
template <typename T> struct Mfma16;
typedef _Float16 ekv_f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 ekv_bf16x8 __attribute__((ext_vector_type(8)));
typedef float ekv_f32x4 __attribute__((ext_vector_type(4)));
template <> struct Mfma16<_Float16> {
  static __device__ __forceinline__ ekv_f32x4 mac(const uint4& a, const uint4& b, ekv_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(ekv_f16x8, a),
                                                  __builtin_bit_cast(ekv_f16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma16<bf16_t> {
  static __device__ __forceinline__ ekv_f32x4 mac(const uint4& a, const uint4& b, ekv_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(ekv_bf16x8, a),
                                                   __builtin_bit_cast(ekv_bf16x8, b), c, 0, 0, 0);
  }
};
template <typename T, int G>
constexpr bool kScoreMfma = (sizeof(T) == 2) && G >= EKV_MFMA_MIN_G;

// score_rows on the matrix cores (see kScoreMfma): every wave scores tiles of
// 16 consecutive compacted tokens, U tiles per round, two rounds in flight.
template <typename T, int LPR, int G, int NT, int U, typename PagePtr>
__device__ __forceinline__ void score_rows_mfma(const DecodeArgs& a, int b, int kvh, int c_begin,
                                                int c_end, float* sc, int64_t stride,
                                                PagePtr pages, int c_base, float* run_max) {
  constexpr int D = LPR * 8;
  constexpr int KB = D / 32;  // 32-wide slices of D
  constexpr int W = NT / 64;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int j = lane & 15;   // A row within the tile; B / C column (query head)
  const int kq = lane >> 4;  // 8-element block within each slice
  const int h0 = kvh * G;
  // B: head j's query (scaled by qscale, rounded to T) at k = 32 i + 8 kq .. +7
  uint4 qb[KB];
  {
    const T* qh = (const T*)a.q + b * a.qsb + (h0 + min(j, G - 1)) * a.qsh;
#pragma unroll
    for (int i = 0; i < KB; ++i) {
      Vec<T> x;
      x.load(qh + 32 * i + 8 * kq);
      T tmp[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) tmp[e] = from_f<T>(j < G ? x.v[e] * a.qscale : 0.f);
      qb[i] = *reinterpret_cast<const uint4*>(tmp);
    }
  }
  float slope = 0.f;
  int q_idx = 0;
  if (a.slopes) {
    q_idx = (a.q_seqlens ? a.q_seqlens[b] : a.cache_seqlens[b * a.csb + kvh * a.csh]) - 1;
    slope = j < G ? a.slopes[h0 + j] * (a.alpha - 1.0f) : 0.f;
  }
  const T* kbase = (const T*)a.k;
  const bool kpos = a.slopes && a.positions;
  const int ps = a.page_size;
  // logical cache row of compacted token c (the ALiBi distance)
  auto row_of = [&](int c) -> int {
    return pages[(c - c_base) / ps] * ps + (c % ps);
  };
  float rmax = -1.0e6f;
  // tile t covers tokens c_begin + 16 t .. + 15; wave wid takes tiles wid + W (u + U m).
  // Lane j (of each 16) resolves token j's row once; the ballot of the
  // valid ones tells the accumulator lanes (token 4 kq + r) which to mask.
  auto fetch = [&](int m, uint4 (&kv)[U][KB], uint64_t (&vm)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c_begin + ((m * U + u) * W + wid) * 16 + j;
      int64_t off = -1;
      if (c < c_end) {
        const int page = pages[(c - c_base) / ps];
        if (page >= 0) off = kv_row_offset(a, b, kvh, (int64_t)page * ps + (c % ps));
      }
      vm[u] = __ballot(off >= 0);
      const T* kr = kbase + (off >= 0 ? off : 0) + 8 * kq;
#pragma unroll
      for (int i = 0; i < KB; ++i) kv[u][i] = ld16(kr + 32 * i);
    }
  };
  auto consume = [&](int m, const uint4 (&kv)[U][KB], const uint64_t (&vm)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      ekv_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < KB; ++i) acc = Mfma16<T>::mac(kv[u][i], qb[i], acc);
      const int t0 = c_begin + ((m * U + u) * W + wid) * 16 + 4 * kq;
      if (j < G) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int c = t0 + r;
          if (c < c_end) {
            float s = acc[r];
            if (!((vm[u] >> (4 * kq + r)) & 1)) s = -INFINITY;
            else if (a.slopes && !kpos) s += slope * (float)(row_of(c) - q_idx);
            sc[j * stride + c] = s;
            if (!kpos) rmax = fmaxf(rmax, s);
          }
        }
      }
    }
  };
  const int tiles = c_end > c_begin ? (c_end - c_begin + 15) / 16 : 0;
  const int rounds = (tiles + U * W - 1) / (U * W);
  uint4 kv_a[U][KB], kv_b[U][KB];
  uint64_t vm_a[U], vm_b[U];
  if (rounds > 0) fetch(0, kv_a, vm_a);
  int r = 0;
  for (; r + 2 < rounds; r += 2) {
    fetch(r + 1, kv_b, vm_b);
    consume(r, kv_a, vm_a);
    fetch(r + 2, kv_a, vm_a);
    consume(r + 1, kv_b, vm_b);
  }
  if (r + 1 < rounds) {
    fetch(r + 1, kv_b, vm_b);
    consume(r, kv_a, vm_a);
    consume(r + 1, kv_b, vm_b);
  } else if (r < rounds) {
    consume(r, kv_a, vm_a);
  }
  if (kpos && j < G) {
    // explicit key positions: the ALiBi term over the scores this lane wrote
    // above (out of the scoring loop, as in score_rows)
    const int32_t* pos = a.positions + b * a.posb + kvh * a.posh;
    for (int m = 0; m < rounds; ++m) {
      for (int u = 0; u < U; ++u) {
        const int t0 = c_begin + ((m * U + u) * W + wid) * 16 + 4 * kq;
        for (int rr = 0; rr < 4; ++rr) {
          const int c = t0 + rr;
          if (c >= c_end) continue;
          const int page = pages[(c - c_base) / ps];
          const int64_t row = (int64_t)page * ps + (c % ps);
          const bool valid = page >= 0 && kv_row_offset(a, b, kvh, row) >= 0;
          float s = sc[j * stride + c];
          if (valid) s += slope * (float)(pos[row] - q_idx);
          sc[j * stride + c] = s;
          rmax = fmaxf(rmax, s);
        }
      }
    }
  }
  if (run_max) {
#pragma unroll
    for (int g = 0; g < G; ++g) run_max[g] = fmaxf(run_max[g], j == g ? rmax : -1.0e6f);
  }
}

// Scores of compacted tokens [c_begin, c_end) of one (b, kv head) for its G
// heads: sc[g * stride + c].  NT threads, rows of LPR lanes, U rows per
// segment in flight.  `pages` holds the page ids of tokens from `c_base` on
// (LDS or global memory).
template <typename T, int LPR, int G, int NT, int U, typename PagePtr>
__device__ __forceinline__ void score_rows(const DecodeArgs& a, int b, int kvh, int c_begin,
                                           int c_end, float* sc, int64_t stride, PagePtr pages,
                                           int c_base, float* run_max = nullptr) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SEGS = NT / LPR;
  constexpr int ROWS = SEGS * U;
  const int seg = threadIdx.x / LPR;
  const int sl = threadIdx.x % LPR;
  const int col = sl * VEC;
  const int h0 = kvh * G;
  if constexpr (kScoreMfma<T, G>) {
    score_rows_mfma<T, LPR, G, NT, 2>(a, b, kvh, c_begin, c_end, sc, stride, pages, c_base,
                                      run_max);
  } else {
  uint4 qraw[G];
  load_query<T, G>(a, b, h0, col, qraw);
  float slope[G];
  int q_idx = 0;
  if (a.slopes) {
    q_idx = (a.q_seqlens ? a.q_seqlens[b] : a.cache_seqlens[b * a.csb + kvh * a.csh]) - 1;
#pragma unroll
    for (int g = 0; g < G; ++g) slope[g] = a.slopes[h0 + g] * (a.alpha - 1.0f);
  }
  const T* kbase = (const T*)a.k;
  const int32_t* kpos = a.slopes && a.positions ? a.positions + b * a.posb + kvh * a.posh : nullptr;
  const int ps = a.page_size;
  constexpr int kNoRow = INT_MIN;
  // Rows of compacted tokens c0 + u * SEGS + seg and their K loads.  The loads
  // are unconditional (an invalid token re-reads row 0 and is masked), so
  // all U of them are in flight together.
  // (generic over the buffer length N: U rows, or 1 for the folded remainder)
  auto fetch = [&](int c0, auto& rows, auto& kv) {
    constexpr int N = sizeof(kv) / sizeof(kv[0]);
    int64_t off[N];
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int c = c0 + u * SEGS + seg;
      rows[u] = kNoRow;
      off[u] = 0;  // an invalid token re-reads the cache's first element
      if (c < c_end) {
        const int page = pages[(c - c_base) / ps];
        const int64_t row = (int64_t)page * ps + (c % ps);
        const int64_t o = page >= 0 ? kv_row_offset(a, b, kvh, row) : -1;
        if (o >= 0) {
          rows[u] = (int)row;
          off[u] = o;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < N; ++u) kv[u] = ld16(kbase + off[u] + col);
  };
  auto consume = [&](int c0, const auto& rows, const auto& kv) {
    constexpr int N = sizeof(kv) / sizeof(kv[0]);
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int c = c0 + u * SEGS + seg;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = Dot16<T>::dot(qraw[g], kv[u], 0.f);
        acc = seg_sum<LPR>(acc);
        if (c < c_end) {
          float s = acc;
          if (rows[u] == kNoRow) s = -INFINITY;
          else if (a.slopes && !kpos) s += slope[g] * (float)(rows[u] - q_idx);
          if (sl == 0) sc[g * stride + c] = s;
          if (run_max && !kpos) run_max[g] = fmaxf(run_max[g], s);
        }
      }
    }
  };
  // two register buffers: the loads of the next round are issued before the
  // current round's arithmetic.  The steady-state loop issues both rounds'
  // loads unconditionally, so the compiler's wait counts keep the other
  // buffer's loads in flight during each consume; the last one or two rounds
  // are peeled.
  // A remainder of at most one row per segment after the full rounds is
  // folded into the first round (loaded with it, scored at the end) instead
  // of costing a round trip of its own: k pages plus a one-token last page
  // (the top-k step after an append) is 2 full rounds and one row.
  int rows_a[U], rows_b[U], rows_x[1];
  uint4 kv_a[U], kv_b[U], kv_x[1];
  const int nrows = c_end > c_begin ? c_end - c_begin : 0;
  const int full = nrows / ROWS, rem = nrows - full * ROWS;
  const bool fold = full > 0 && rem > 0 && rem <= SEGS;
  const int rounds = fold ? full : (nrows + ROWS - 1) / ROWS;
  if (rounds > 0) fetch(c_begin, rows_a, kv_a);
  if (fold) fetch(c_begin + full * ROWS, rows_x, kv_x);
  int r = 0;
  for (; r + 2 < rounds; r += 2) {
    fetch(c_begin + (r + 1) * ROWS, rows_b, kv_b);
    consume(c_begin + r * ROWS, rows_a, kv_a);
    fetch(c_begin + (r + 2) * ROWS, rows_a, kv_a);
    consume(c_begin + (r + 1) * ROWS, rows_b, kv_b);
  }
  if (r + 1 < rounds) {
    fetch(c_begin + (r + 1) * ROWS, rows_b, kv_b);
    consume(c_begin + r * ROWS, rows_a, kv_a);
    consume(c_begin + (r + 1) * ROWS, rows_b, kv_b);
  } else if (r < rounds) {
    consume(c_begin + r * ROWS, rows_a, kv_a);
  }
  if (fold) consume(c_begin + full * ROWS, rows_x, kv_x);
  if (kpos && sl == 0) {
    // explicit key positions: the ALiBi term (and the running max) over the
    // scores this lane wrote above (lane 0 of each row segment: it alone
    // reads back its own stores); kept out of the scoring loop, whose K
    // loads would otherwise all drain before every position load's use.  The
    // running max is reduced over all lanes later, so lane 0 carries it.
    for (int c = c_begin + seg; c < c_end; c += SEGS) {
      const int page = pages[(c - c_base) / ps];
      const int64_t row = (int64_t)page * ps + (c % ps);
      const bool valid = page >= 0 && kv_row_offset(a, b, kvh, row) >= 0;
      const float bias = valid ? (float)(kpos[valid ? row : 0] - q_idx) : 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float s = sc[g * stride + c];
        if (valid) s += slope[g] * bias;
        sc[g * stride + c] = s;
        if (run_max) run_max[g] = fmaxf(run_max[g], s);
      }
    }
  }
  }
}

// ---------------------------------------------------------------------------
// tau: kernels/adadecode.py:12-112, 381-426, 555-592 and
// kernels/adadecode_paged_gaussian_tau.py:12-53
// ---------------------------------------------------------------------------

__device__ __forceinline__ void histogram_init_vals(const int (&hv)[kBins], float gmax, float alpha,
                                                    float& t, float& t_lo, float& t_hi) {
  const float t0 = gmax - 1.0f;
  if (alpha == 2.0f || alpha == 1.5f) {
    float sum_z = 1.f, sum_k = 1.f, sum_z2 = 1.f;
#pragma unroll
    for (int sj = kBins - 1; sj >= 0; --sj) {
      float c_bin = (float)hv[sj];
      if (sj == kBins - 1) c_bin -= 1.0f;
      const float c_tau = (float)sj / (float)kBins;
      const float new_z = sum_z + c_bin * c_tau;
      const float new_k = sum_k + c_bin;
      if (alpha == 2.0f) {
        if ((new_z - new_k * c_tau) < 1.0f) {
          sum_z = new_z;
          sum_k = new_k;
        }
      } else {
        const float new_z2 = sum_z2 + c_bin * (c_tau * c_tau);
        if (new_k * c_tau * c_tau - 2.0f * new_z * c_tau + new_z2 < 1.0f) {
          sum_z = new_z;
          sum_k = new_k;
          sum_z2 = new_z2;
        }
      }
    }
    float t_init;
    if (alpha == 2.0f) {
      t_init = gmax + (sum_z - 1.0f) / sum_k - 1.0f;
    } else {
      const float disc = sum_z * sum_z - sum_k * (sum_z2 - 1.0f);
      t_init = gmax + (sum_z - sqrtf(disc)) / sum_k - 1.0f;
    }
    t_lo = t_init;
    t_hi = t_init + 1.0f / kBins;
  } else {
    const float p = 1.0f / (alpha - 1.0f);
    int lo = 0, hi = kBins - 1, found = 0, b_idx = 0;
    for (int it = 0; it < 5; ++it) {
      const int mid = (int)((float)(lo + hi) * 0.5f);
      float fL = 0.f, fU = 0.f;
#pragma unroll
      for (int j = 0; j < kBins; ++j) {
        const int off = j - mid;
        if (off < 0) continue;
        float cnt = (float)hv[j];
        if (j == kBins - 1) cnt -= 1.0f;
        const float zL = (float)off / kBins;
        const float zU = ((float)off + 1.0f) / kBins;
        if (zL > 0.f) fL += cnt * exp2f(log2f(zL) * p);
        fU += cnt * exp2f(log2f(zU) * p);
      }
      fL -= 1.0f;
      fU -= 1.0f;
      const bool go_right = fL > 0.f, go_left = fU < 0.f;
      const bool bracket = !go_right && !go_left;
      if (found == 0) {
        if (bracket) {
          b_idx = mid;
          found = 1;
        }
        if (go_right) lo = mid + 1;
        if (go_left) hi = mid - 1;
      }
    }
    const int b_sel = found ? b_idx : min(lo, kBins - 1);
    t_lo = t0 + (float)b_sel / kBins;
    t_hi = t0 + (float)min(b_sel + 1, kBins) / kBins;
  }
  t = 0.5f * (t_lo + t_hi);
}

__device__ __forceinline__ void histogram_init(const int* hist, float gmax, float alpha, float& t,
                                               float& t_lo, float& t_hi) {
  // all bins in registers first (one LDS round trip instead of one per bin)
  int hv[kBins];
  const int4* h4 = reinterpret_cast<const int4*>(hist);
#pragma unroll
  for (int j = 0; j < kBins / 4; ++j) {
    const int4 x = h4[j];
    hv[4 * j] = x.x;
    hv[4 * j + 1] = x.y;
    hv[4 * j + 2] = x.z;
    hv[4 * j + 3] = x.w;
  }
  histogram_init_vals(hv, gmax, alpha, t, t_lo, t_hi);
}

// Token counts up to which the bin sums of histogram_init_wave are exact in
// fp32 (sum of count * bin^2 below 2^24).
constexpr int kExactInitTokens = 65536;

// histogram_init over bin counts that lane j (j < kBins) of the wave holds
// for bin kBins - 1 - j, alpha 2 and 1.5 only: every lane takes the suffix
// sums of the bins from the top down to its own (exact integer prefix sums
// scaled by 1/16 and 1/256, so every sum and every test below is exact in
// fp32 for the token counts of this path and equals the serial loop of
// histogram_init), the accepted bins are the top run whose test holds (the
// test is monotone in the bin), and the sums of its lowest bin give t.
__device__ __forceinline__ void histogram_init_wave(int cnt_rev, float gmax, float alpha,
                                                    float& t, float& t_lo, float& t_hi) {
  const int lane = threadIdx.x & 63;
  const int sj = kBins - 1 - lane;  // this lane's bin
  const int c = lane < kBins ? cnt_rev - (lane == 0 ? 1 : 0) : 0;
  const int ik = wave_incl_scan(c);
  const int iz = wave_incl_scan(c * sj);
  const int iz2 = wave_incl_scan(c * sj * sj);
  const float c_tau = (float)sj / (float)kBins;
  const float new_z = 1.0f + (float)iz / (float)kBins;
  const float new_k = 1.0f + (float)ik;
  const float new_z2 = 1.0f + (float)iz2 / (float)(kBins * kBins);
  bool ok;
  if (alpha == 2.0f) {
    ok = (new_z - new_k * c_tau) < 1.0f;
  } else {
    ok = new_k * c_tau * c_tau - 2.0f * new_z * c_tau + new_z2 < 1.0f;
  }
  const uint64_t acc = __ballot(lane < kBins && ok);
  const int m = (int)__builtin_ctzll(~acc);  // accepted bins: lanes 0 .. m-1
  float sum_z = 1.f, sum_k = 1.f, sum_z2 = 1.f;
  if (m > 0) {
    sum_z = __shfl(new_z, m - 1);
    sum_k = __shfl(new_k, m - 1);
    sum_z2 = __shfl(new_z2, m - 1);
  }
  float t_init;
  if (alpha == 2.0f) {
    t_init = gmax + (sum_z - 1.0f) / sum_k - 1.0f;
  } else {
    const float disc = sum_z * sum_z - sum_k * (sum_z2 - 1.0f);
    t_init = gmax + (sum_z - sqrtf(disc)) / sum_k - 1.0f;
  }
  t_lo = t_init;
  t_hi = t_init + 1.0f / kBins;
  t = 0.5f * (t_lo + t_hi);
}

__device__ __forceinline__ void halley_bisect(float& t, float& t_lo, float& t_hi, float a0,
                                              float a1, float a2, float c0, float c1) {
  const float ff = a0 - 1.0f;
  const float df = -c0 * a1;
  const float ddf = c0 * c1 * a2;
  if (ff > 0.f) t_lo = t;
  if (ff < 0.f) t_hi = t;
  const float new_t = t - (2.f * ff * df) / (2.f * df * df - ff * ddf);
  const bool good = (new_t > t_lo - 1e-6f) && (new_t < t_hi + 1e-6f);
  t = good ? new_t : 0.5f * (t_lo + t_hi);
}

__device__ __forceinline__ float halley_unbounded(float t, float a0, float a1, float a2, float c0,
                                                  float c1) {
  const float ff = a0 - 1.0f;
  const float df = -c0 * a1;
  const float ddf = c0 * c1 * a2;
  const float hden = 2.0f * df * df - ff * ddf;
  float tn;
  if (fabsf(hden) > 1e-12f) tn = t - (2.0f * ff * df) / hden;
  else if (fabsf(df) > 1e-12f) tn = t - ff / df;
  else tn = t;
  if (!(tn == tn && fabsf(tn) < 1e20f)) tn = t;
  return tn;
}

// Reduction scope of a tau solve: a team of W consecutive waves owns one head
// (lanes stride 64 * W).  W = 1 needs no workgroup barrier; for W > 1 every
// wave of the workgroup makes the same sequence of reductions (a wave without
// a head runs the solve on zero scores), and the partials of each reduction
// go through one of two LDS buffers in turn, so one barrier per reduction
// suffices.
template <int W>
struct TeamScope {
  static constexpr int kStride = 64 * W;
  float4* part;  // [2][kWaves] per-wave partials (LDS)
  int wid, lane, team, pos, parity;
  __device__ __forceinline__ TeamScope(float4* p) : part(p), parity(0) {
    wid = threadIdx.x >> 6;
    lane = threadIdx.x & 63;
    team = wid / W;
    pos = wid % W;
  }
  __device__ __forceinline__ int first() const { return pos * 64 + lane; }
  __device__ __forceinline__ void sync() const {
    if constexpr (W == 1) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    } else {
      __syncthreads();
    }
  }
  __device__ __forceinline__ float max(float x) {
    x = wave_max(x);
    if constexpr (W > 1) {
      float4* buf = part + parity * kWaves;
      if (lane == 0) buf[wid].x = x;
      __syncthreads();
      x = buf[team * W].x;
#pragma unroll
      for (int w = 1; w < W; ++w) x = fmaxf(x, buf[team * W + w].x);
      parity ^= 1;
    }
    return x;
  }
  __device__ __forceinline__ void sum3(float& a, float& b, float& c) {
    a = wave_sum(a);
    b = wave_sum(b);
    c = wave_sum(c);
    if constexpr (W > 1) {
      float4* buf = part + parity * kWaves;
      if (lane == 0) buf[wid] = make_float4(a, b, c, 0.f);
      __syncthreads();
      float4 r = buf[team * W];
#pragma unroll
      for (int w = 1; w < W; ++w) {
        const float4 y = buf[team * W + w];
        r.x += y.x;
        r.y += y.y;
        r.z += y.z;
      }
      a = r.x;
      b = r.y;
      c = r.z;
      parity ^= 1;
    }
  }
};

// One pass over scores[0..n) of a head: the sums of [s - t]_+^(1/(alpha-1) - j)
// for j = 0, 1, 2 (kernels/adadecode_paged.py:357-372), branch-free per score.
template <typename S>
__device__ __forceinline__ void accumulate_pass(S& sp, const float* __restrict__ sc, int n, float t,
                                                float alpha, float c0, float& a0, float& a1,
                                                float& a2) {
  float s0 = 0.f, s1 = 0.f, s2 = 0.f;
  const bool generic = !(alpha == 2.0f || alpha == 1.5f);
  const bool sparsemax = alpha == 2.0f;
  for (int b0 = 0; b0 < n; b0 += S::kStride * kBatch) {
    float x[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) {
      const int c = b0 + j * S::kStride + sp.first();
      x[j] = c < n ? sc[c] : -INFINITY;
    }
    if (!generic) {
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const bool act = x[j] > t;
        const float d = act ? x[j] - t : 0.f;
        const float one = act ? 1.f : 0.f;
        s0 += sparsemax ? d : d * d;
        s1 += sparsemax ? one : d;
        s2 += sparsemax ? 0.f : one;
      }
    } else {
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        if (x[j] > t) {
          const float l = log2f(x[j] - t);
          s0 += exp2f(l * c0);
          s1 += exp2f(l * (c0 - 1.f));
          s2 += exp2f(l * (c0 - 2.f));
        }
      }
    }
  }
  sp.sum3(s0, s1, s2);
  a0 = s0;
  a1 = s1;
  a2 = s2;
}

// tau of one head (kernels/adadecode_paged.py:140-247, 357-372 and
// kernels/adadecode_paged_gaussian_tau.py:12-53).  `hist` (kBins ints, LDS)
// must be zero on entry when tau_mode is 0.
template <typename S>
__device__ __forceinline__ float solve_tau(S& sp, const DecodeArgs& a, const float* __restrict__ sc,
                                           int n, float tau_in, int* hist, const float* pre_max) {
  const float alpha = a.alpha;
  const float c0 = 1.0f / (alpha - 1.0f);
  const float c1 = c0 - 1.0f;
  float t;
  if (a.tau_mode == 0) {
    float m = -1.0e6f;
    // the max of the scores, from the scoring phase when it ran in this launch
    if (pre_max) {
      m = *pre_max;
    } else for (int b0 = 0; b0 < n; b0 += S::kStride * kBatch) {
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int c = b0 + j * S::kStride + sp.first();
        if (c < n) m = fmaxf(m, sc[c]);
      }
    }
    const float gmax = pre_max ? m : sp.max(m);
    EKV_TSTAMP(7);
    const float t0 = gmax - 1.0f;
    for (int b0 = 0; b0 < n; b0 += S::kStride * kBatch) {
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int c = b0 + j * S::kStride + sp.first();
        if (c < n) {
          const float f = (sc[c] - t0) * (float)kBins;
          if (f > -1.0f) atomicAdd(&hist[min((int)f, kBins - 1)], 1);
        }
      }
    }
    sp.sync();
    EKV_TSTAMP(8);
    float t_lo, t_hi;
    if ((alpha == 2.0f || alpha == 1.5f) && n <= kExactInitTokens)
      histogram_init_wave(hist[kBins - 1 - min(sp.lane, kBins - 1)], gmax, alpha, t, t_lo, t_hi);
    else
      histogram_init(hist, gmax, alpha, t, t_lo, t_hi);
    EKV_TSTAMP(9);
    for (int it = 0; it < a.iters; ++it) {
      float a0, a1, a2;
      accumulate_pass(sp, sc, n, t, alpha, c0, a0, a1, a2);
      halley_bisect(t, t_lo, t_hi, a0, a1, a2, c0, c1);
      if (it < 2) EKV_TSTAMP(10 + it);
    }
  } else {
    t = tau_in;
    for (int it = 0; it < a.iters; ++it) {
      float a0, a1, a2;
      accumulate_pass(sp, sc, n, t, alpha, c0, a0, a1, a2);
      t = halley_unbounded(t, a0, a1, a2, c0, c1);
    }
  }
  return t;
}

// ---------------------------------------------------------------------------
// phase 1 as its own launch (few heads)
// ---------------------------------------------------------------------------

template <typename T, int LPR, int G>
__global__ __launch_bounds__(kSplitThreads) void score_split_kernel(DecodeArgs a) {
  const int split = blockIdx.x;
  const int bkv = blockIdx.y;
  const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
  const int n = token_count(a, b, kvh);
  const int per = (n + a.splits - 1) / a.splits;
  const int c_start = split * per;
  const int c_end = min(c_start + per, n);
  if (c_start >= c_end) return;
  float* sc = a.ws_scores + ((int64_t)b * a.H + kvh * G) * a.max_tokens;
  const int32_t* pi = a.page_indices + b * a.pisb + kvh * a.pish;
  // The page ids come from LDS, a chunk at a time: read from global memory
  // inside the loop, each one would wait behind the K loads already in flight
  // (vector loads complete in order), which drains the second register buffer.
  __shared__ int s_pages[kSplitTablePages];
  const int ps = a.page_size;
  for (int cb = c_start; cb < c_end;) {
    const int p0 = cb / ps;
    const int ce = min(c_end, (p0 + kSplitTablePages) * ps);
    const int np = (ce - 1) / ps - p0 + 1;
    __syncthreads();  // the previous chunk's readers are done
    for (int i = threadIdx.x; i < np; i += kSplitThreads) s_pages[i] = pi[p0 + i];
    __syncthreads();
    score_rows<T, LPR, G, kSplitThreads, kSplitUnroll>(a, b, kvh, cb, ce, sc, a.max_tokens,
                                                       (const int*)s_pages, p0 * ps);
    cb = ce;
  }
}

// ---------------------------------------------------------------------------
// the head kernel
// ---------------------------------------------------------------------------

struct HeadShared {
  int (*hist)[kBins];
  float4* part;  // [2][kWaves] reduction partials
  float* s_tau;
  int* sup_row;  // [sup_chunk(G)] V rows of the support (rows of ksr elements from the base)
  float* sup_p;  // [G][sup_chunk(G)]
  int* flag_cnt;
  float* red;    // [kWaves][D]
  int* s_pages;  // [kTablePages]
  const float* tau_in_lds = nullptr;  // [G] starting tau in LDS (else a.tau_in)
  float* wmax = nullptr;              // [G][kWaves] per-wave score maxima of phase 1
};

// tau of the G heads of one (b, kv head): head g is solved by the team of W
// waves g * W .. g * W + W - 1 (short token lists: W = 4 / G, one wave per
// SIMD; long ones: every wave of the workgroup).
template <int W, int G>
__device__ __forceinline__ void solve_heads(const DecodeArgs& a, int b, int h0, int n,
                                            const float* sc, int64_t stride,
                                            const HeadShared& sh) {
  TeamScope<W> sp(sh.part);
  const int g = sp.team;
  if (W == 1 && g >= G) return;
  const bool real = g < G;
  float tin = 0.f;
  if (real && a.tau_mode == 1) tin = sh.tau_in_lds ? sh.tau_in_lds[g] : a.tau_in[b * a.H + h0 + g];
  // every team takes the same path (the reductions of a team of W > 1 waves
  // are workgroup barriers)
  float pm = -1.0e6f;
  if (sh.wmax && real)
    for (int w = 0; w < kWaves; ++w) pm = fmaxf(pm, sh.wmax[g * kWaves + w]);
  const float t = solve_tau(sp, a, sc + (real ? g : 0) * stride, real ? n : 0, tin, sh.hist[g],
                            sh.wmax ? &pm : nullptr);
  if (real && sp.pos == 0 && sp.lane == 0) sh.s_tau[g] = t;
}

// Two workgroups per (b, kv head) (the paired Gaussian launch): each scored
// the tokens [c0, c1) of the head's n into `sc` (LDS, or the head's workspace
// row).  Each stores them to the workspace with agent-scope stores (written
// through to the level every XCD reads; a waitcnt completes them) and
// exchanges the launch's tag into the pair's word: the first to arrive
// returns false and is done; the second sets the word back to zero, loads its
// partner's scores with agent-scope loads into `sc` (in the workspace case
// storing them back with plain stores, so that its later plain loads see
// them whatever its L2 holds), folds them into the per-wave maxima and
// returns true to solve tau and gather V for the head.
template <int G>
__device__ __forceinline__ bool pair_handoff(const DecodeArgs& a, int b, int h0, int n, int c0,
                                             int c1, float* sc, int64_t stride,
                                             const HeadShared& sh, unsigned long long* word,
                                             unsigned long long tag) {
  const int tid = threadIdx.x;
  float* ws = a.ws_scores + ((int64_t)b * a.H + h0) * a.max_tokens;
#pragma unroll
  for (int g = 0; g < G; ++g)
    for (int c = c0 + tid; c < c1; c += kHeadThreads)
      __hip_atomic_store(ws + (int64_t)g * a.max_tokens + c, sc[g * stride + c], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const unsigned long long old =
        __hip_atomic_exchange(word, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == tag) __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh.flag_cnt[0] = old == tag ? 1 : 0;
  }
  __syncthreads();
  if (sh.flag_cnt[0] == 0) return false;
  const int p0 = c0 == 0 ? c1 : 0, p1 = c0 == 0 ? n : c0;
  float m[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -1.0e6f;
    for (int c = p0 + tid; c < p1; c += kHeadThreads) {
      const float v = __hip_atomic_load(ws + (int64_t)g * a.max_tokens + c, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
      sc[g * stride + c] = v;
      m[g] = fmaxf(m[g], v);
    }
  }
  if (sh.wmax) {
    const int lane = tid & 63, wid = tid >> 6;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float w = wave_max(m[g]);
      if (lane == 0) sh.wmax[g * kWaves + wid] = fmaxf(sh.wmax[g * kWaves + wid], w);
    }
  }
  __syncthreads();
  return true;
}

// Phases 1-3 of one (b, kv head); `sc` points to LDS when kStaged (so every
// score access is a ds_* instruction) and to the workspace otherwise.
template <typename T, int LPR, int G, int U, bool kStaged, bool kTableInLds = false>
__device__ __forceinline__ bool decode_head_body(const DecodeArgs& a, int b, int kvh, int n,
                                                 float* sc, int64_t stride,
                                                 const HeadShared& sh_in,
                                                 bool first_chunk_staged = false,
                                                 unsigned long long* pair_word = nullptr,
                                                 unsigned long long pair_tag = 0,
                                                 int pair_half = 0) {
  // the per-wave maxima reach the tau solve only when phase 1 runs here
  HeadShared sh = sh_in;
  if (a.scores_ready && !kTableInLds) sh.wmax = nullptr;
  constexpr int VEC = 16 / sizeof(T);
  constexpr int SEGS = kHeadThreads / LPR;
  constexpr int D = LPR * VEC;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const int h0 = kvh * G;
  const int ps = a.page_size;
  const int32_t* pi = a.page_indices + b * a.pisb + kvh * a.pish;
  if (tid < kWaves * kBins) (&sh.hist[0][0])[tid] = 0;  // read after the phase-1 barriers
  // phase 1: scores (and each head's running max), the page table staged in
  // LDS chunk by chunk
  float rmax[G];
#pragma unroll
  for (int g = 0; g < G; ++g) rmax[g] = -1.0e6f;
  // paired: this workgroup scores the first or the second half of the tokens
  // (split on a multiple of 64 tokens, and of 64 pages when the page table is
  // staged chunk by chunk)
  int pc0 = 0, pc1 = n;
  if (pair_word) {
    const int q = kTableInLds ? 64 : 64 * ps;
    const int mid = min(n, (n / 2 + q - 1) / q * q);
    if (pair_half) pc0 = mid;
    else pc1 = mid;
  }
  if (kTableInLds) {
    // the whole page table is already in sh.s_pages (written by this workgroup)
    score_rows<T, LPR, G, kHeadThreads, U>(a, b, kvh, pc0, pc1, sc, stride, sh.s_pages, 0, rmax);
  } else if (!a.scores_ready) {
    for (int cb = pc0; cb < pc1; cb += kTablePages * ps) {
      const int ce = min(pc1, cb + kTablePages * ps);
      const int np = (ce - cb + ps - 1) / ps;
      if (!(first_chunk_staged && cb == 0)) {
        for (int i = tid; i < np; i += kHeadThreads) sh.s_pages[i] = pi[cb / ps + i];
      }
      __syncthreads();
      score_rows<T, LPR, G, kHeadThreads, U>(a, b, kvh, cb, ce, sc, stride, sh.s_pages, cb,
                                             rmax);
      __syncthreads();
    }
  }
  if (sh.wmax) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float m = wave_max(rmax[g]);
      if (lane == 0) sh.wmax[g * kWaves + wid] = m;
    }
  }
  EKV_WSTAMP(5);
  __syncthreads();
  if (pair_word && !pair_handoff<G>(a, b, h0, n, pc0, pc1, sc, stride, sh, pair_word, pair_tag))
    return false;
  EKV_STAMP(3);

  // phase 2: tau per head, one team of waves per head: for lists up to 4096
  // tokens 4 / G waves (one per SIMD; G = 1 at the headline shape: teams of 1,
  // 2, 4 and 8 waves took 67.3, 67.0, 66.2 and 66.8 us per step), or kWaves /
  // G for G >= 4 (config 4: 4 waves per head 133.2 us against one wave 135.1
  // us); the whole workgroup for longer lists
  constexpr int kTeam = G >= 4 ? kWaves / G : 4 / G;
  if (n <= 4096) {
    solve_heads<kTeam, G>(a, b, h0, n, sc, stride, sh);
  } else {
    solve_heads<kWaves / G, G>(a, b, h0, n, sc, stride, sh);
  }
  __syncthreads();
  float tau[G];
#pragma unroll
  for (int g = 0; g < G; ++g) tau[g] = sh.s_tau[g];
  if (tid < G) a.tau[b * a.H + h0 + tid] = sh.s_tau[tid];
  EKV_STAMP(4);

  // phase 3: gather the support's V rows
  const float alpha = a.alpha;
  const float c0 = 1.0f / (alpha - 1.0f);
  const int seg = tid / LPR;
  const int col = (tid % LPR) * VEC;
  const T* vbase = (const T*)a.v;
  float acc[G][VEC];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[g][i] = 0.f;

  // The support is compacted a chunk of TPT * kHeadThreads tokens at a time
  // (TPT tokens per thread; one chunk covers the selections of the common
  // shapes), and only its V rows are read.  The scores (and, from global
  // memory, the page ids) of the next chunk are loaded before this chunk's V
  // rows, so they have landed when the chunk after starts (the loads are
  // clamped to the last token and issued unconditionally).
  constexpr int TPT = sup_chunk(G) / kHeadThreads;
  constexpr int CH = sup_chunk(G);
  float s_nx[TPT][G];
  int pg_nx[TPT];
  auto prefetch = [&](int t0) {
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      const int cc = min(t0 + j * kHeadThreads + tid, n - 1);
#pragma unroll
      for (int g = 0; g < G; ++g) s_nx[j][g] = sc[g * stride + cc];
      pg_nx[j] = kTableInLds ? 0 : pi[cc / ps];
    }
  };
  if (n > 0) prefetch(0);
  for (int t0 = 0; t0 < n; t0 += CH) {
    float p[TPT][G];
    bool any[TPT];
    int row[TPT];
    uint64_t m[TPT];
    int mine = 0;
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      const int c = t0 + j * kHeadThreads + tid;
      any[j] = false;
      row[j] = -1;
      if (c < n) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float sv = s_nx[j][g];
          p[j][g] = 0.f;
          if (sv > tau[g]) {
            p[j][g] = entmax_weight(sv - tau[g], alpha, c0);
            any[j] = true;
          }
        }
        if (any[j]) {
          int64_t r;
          if (kTableInLds) {
            r = token_row(sh.s_pages, c, ps, a.row_limit);
          } else {
            const int pg = pg_nx[j];
            r = (int64_t)pg * ps + (c % ps);
            r = (pg >= 0 && r < a.row_limit) ? r : -1;
          }
          // the row's place in V, in rows of ksr elements from the base
          const int64_t o = r >= 0 ? kv_row_offset(a, b, kvh, r) : -1;
          row[j] = (int)(o / a.ksr);
          if (o < 0) any[j] = false;
        }
      }
      m[j] = __ballot(any[j]);
      mine += __popcll(m[j]);
    }
    if (t0 + CH < n) prefetch(t0 + CH);
    if (lane == 0) sh.flag_cnt[wid] = mine;
    __syncthreads();
    int before = 0, nsup = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const int cw = sh.flag_cnt[w];
      before += (w < wid) ? cw : 0;
      nsup += cw;
    }
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int j = 0; j < TPT; ++j) {
      if (any[j]) {
        const int slot = before + __popcll(m[j] & below);
        sh.sup_row[slot] = row[j];
#pragma unroll
        for (int g = 0; g < G; ++g) sh.sup_p[g * CH + slot] = p[j][g];
      }
      before += __popcll(m[j]);
    }
    __syncthreads();
    // eight support rows per segment in flight, kept raw until converted (a
    // slot past nsup re-reads the last row and is not accumulated)
    constexpr int R = 8;
    for (int j0 = seg; j0 < nsup; j0 += R * SEGS) {
      uint4 x[R];
#pragma unroll
      for (int r = 0; r < R; ++r)
        x[r] = ld16(vbase + (int64_t)sh.sup_row[min(j0 + r * SEGS, nsup - 1)] * a.ksr + col);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int j = j0 + r * SEGS;
        if (j < nsup) {
          const T* e = reinterpret_cast<const T*>(&x[r]);
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float w = sh.sup_p[g * CH + j];
#pragma unroll
            for (int i = 0; i < VEC; ++i) acc[g][i] += w * to_f<T>(e[i]);
          }
        }
      }
    }
    __syncthreads();
  }
  EKV_STAMP(5);

  // reduce the row segments: within each wave by shuffles, then across waves
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      acc[g][i] = lanes::cross_seg_sum<LPR>(acc[g][i]);
    }
    if (lane < LPR) {
#pragma unroll
      for (int i = 0; i < VEC; ++i) sh.red[wid * D + col + i] = acc[g][i];
    }
    __syncthreads();
    for (int e = tid; e < D; e += kHeadThreads) {
      float r = 0.f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) r += sh.red[w * D + e];
      T* o = (T*)a.out + b * a.osb + (h0 + g) * a.osh;
      o[e] = from_f<T>(r);
    }
    __syncthreads();
  }
  return true;
}

template <typename T, int LPR, int G, int U>
__global__ __launch_bounds__(kHeadThreads) void decode_head_kernel(DecodeArgs a) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int D = LPR * VEC;
  extern __shared__ __attribute__((aligned(16))) float stage[];  // [G][stage_cap] scores when staged
  __shared__ __attribute__((aligned(16))) int hist[kWaves][kBins];
  __shared__ float4 part[2 * kWaves];
  __shared__ float s_tau[G];
  __shared__ int sup_row[sup_chunk(G)];
  __shared__ float sup_p[G * sup_chunk(G)];
  __shared__ int flag_cnt[kWaves];
  __shared__ float red[kWaves * D];
  __shared__ int s_pages[kTablePages];
  __shared__ float wmax[G * kWaves];
  HeadShared sh{hist, part, s_tau, sup_row, sup_p, flag_cnt, red, s_pages};
  sh.wmax = wmax;

  const int bkv = blockIdx.x;
  const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
  const int n = token_count(a, b, kvh);
  if (!a.scores_ready && n <= a.stage_cap) {
    decode_head_body<T, LPR, G, U, true>(a, b, kvh, n, stage, a.stage_cap, sh);
  } else {
    float* ws = a.ws_scores + ((int64_t)b * a.H + kvh * G) * a.max_tokens;
    decode_head_body<T, LPR, G, U, false>(a, b, kvh, n, ws, a.max_tokens, sh);
  }
}

// Criticality scan + top-k page selection of one step, as read by the fused
// kernel (see ekv_topk_paged_entmax_decode).
struct SelectArgs {
  const void* kmin;
  const void* kmax;
  int64_t ssb, ssh, ssp;
  void* scores;       // [B, H, num_pages] query dtype
  int num_pages;      // pages scored (the last, partial page excluded)
  int seq_len, q_pos;
  int k;              // pages selected per (b, kv head)
  int last_page;      // appended at slot k (the sentinel), or -1
  int key_cap;        // page keys that fit the dynamic LDS
  int head_keys;      // G > 1: every query head's page keys kept in LDS too
  int list_words;     // G > 1: LDS words of the candidate lists
  int prescored;      // the scores are already in `scores` (a split scan ran first)
  // fused append (uniform batch): row app_pos of K and V from app_k / app_v
  // [B, Hkv, D] rows (strides app_nsb, app_nsh) and the four statistics of
  // its page (kmin, kmax above; app_kmean, app_kstd with the same strides),
  // before anything reads them; app_k null: no append
  const void* app_k = nullptr;
  const void* app_v = nullptr;
  int64_t app_nsb = 0, app_nsh = 0;
  void* app_kmean = nullptr;
  void* app_kstd = nullptr;
  int app_pos = -1;
  const int32_t* seq_lens;  // [B] per-sequence lengths (ragged batch) or null
  int scan_rev = 0;         // the scan hands out its page chunks last first
  int scan_nt = 0;          // the scan's loads are non-temporal (stream_nt)
  // the paired launch (2 B Hkv <= CUs, G <= 2, every head's keys in LDS): two
  // workgroups per (b, kv head), each scanning half of the pages, with one
  // arrival word per pair (any value on entry that is not pair_tag; left 0)
  unsigned long long* pair_cnt = nullptr;
  unsigned long long pair_tag = 0;
};

// One (b, kv head) per workgroup end to end: criticality scan of every page
// (or, when t.prescored, the scores a split scan over every CU wrote), top-k
// (page table to global memory and to LDS), then phases 1-3 of the decode on
// the selected pages.  Keys and then scores share the dynamic LDS.
//
// kPair: two workgroups per (b, kv head) scan one half of its pages
// each, storing their scores with store_through, and count their arrival by
// exchanging t.pair_tag into the pair's word (a fresh tag per launch, so a
// stale word never matches, and the second to arrive sets it back to zero,
// so a replayed graph with the same tag starts clean).  The first to arrive
// leaves; the second loads its partner's half of the scores with
// load_through, adds their keys to its LDS keys (G == 1: and first-digit
// histogram; G > 1: every query head's keys, which the launch must keep in
// LDS), and selects and decodes as a lone workgroup would.  The scores of every page are
// computed alone, so the results are those of the one-workgroup launch.
template <typename T, int LPR, int G, int UC, int UD, bool kPair = false>
__global__ __launch_bounds__(kHeadThreads) void topk_decode_kernel(DecodeArgs a, SelectArgs t) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int D = LPR * VEC;
  extern __shared__ __attribute__((aligned(16))) float stage[];
  __shared__ __attribute__((aligned(16))) int hist[kWaves][kBins];
  __shared__ float4 part[2 * kWaves];
  __shared__ float s_tau[G];
  __shared__ int sup_row[sup_chunk(G)];
  __shared__ float sup_p[G * sup_chunk(G)];
  __shared__ int flag_cnt[kWaves];
  __shared__ float red[kWaves * D];
  __shared__ int s_pages[kTablePages];
  __shared__ float wmax[G * kWaves];
  // G == 1: the select's radix histograms; the scan fills the first
  __shared__ unsigned sel_hist[G == 1 ? topk::ScoreKey<T>::kBits / 8 : 1][256];
  HeadShared sh{hist, part, s_tau, sup_row, sup_p, flag_cnt, red, s_pages};
  sh.wmax = wmax;

  const int bkv = kPair ? blockIdx.x >> 1 : blockIdx.x;
  const int pair_half = kPair ? blockIdx.x & 1 : 0;
  const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
  uint32_t* keys = reinterpret_cast<uint32_t*>(stage);
  // the scan's chunk counter (and, G == 1, the select's histograms) start at zero
  __shared__ int scan_next;
  if (threadIdx.x == 0) scan_next = 0;
  if (G == 1) {
    for (int i = threadIdx.x; i < (int)(sizeof(sel_hist) / 4); i += kHeadThreads)
      (&sel_hist[0][0])[i] = 0u;
  }
  if (G == 1 || !t.prescored) __syncthreads();
  if (t.app_k && threadIdx.x < LPR) {
    // the appended row and its page's statistics: the page is the last one,
    // which the scan never reads; the K/V phases read the row after the
    // select's barriers.  The first wave joins the scan afterwards (its
    // chunks go to the others meanwhile).
    const int pos = t.app_pos;
    const int64_t o0 = kv_row_offset(a, b, kvh, (int64_t)(pos / a.page_size) * a.page_size);
    if (o0 >= 0) {
      const int64_t shift = o0 - (int64_t)(pos / a.page_size) * a.page_size * a.ksr;
      const int64_t so = b * t.ssb + kvh * t.ssh + (int64_t)(pos / a.page_size) * t.ssp;
      PageStatRows<T> rows{(T*)t.kmin + so, (T*)t.kmax + so, (T*)t.app_kmean + so,
                           (T*)t.app_kstd + so};
      append_row<T, LPR>((const T*)t.app_k + b * t.app_nsb + kvh * t.app_nsh,
                         (const T*)t.app_v + b * t.app_nsb + kvh * t.app_nsh,
                         (T*)a.k + shift, (T*)a.v + shift, a.ksr, pos, a.page_size, rows,
                         (int)threadIdx.x * VEC);
    }
  }
  const topk::Ragged r = topk::ragged_topk(t.seq_lens, b, a.page_size, t.num_pages, t.seq_len,
                                           t.q_pos, t.k, t.last_page);
  const bool keep = r.count <= t.key_cap;
  // G > 1: [page ranks: num_pages][candidate lists: list_words][head keys: G * num_pages]
  uint32_t* list = keys + t.num_pages;
  uint32_t* head_keys = G > 1 && t.head_keys ? list + t.list_words : nullptr;
  EKV_STAMP(0);
  const T* sbase = (const T*)t.scores + ((int64_t)b * a.H + kvh * G) * t.num_pages;
  // kPair: this workgroup's half of the pages [pp0, pp1) (split on a chunk)
  int pp0 = 0, pp1 = r.count;
  if constexpr (kPair) {
    constexpr int kChunk = UC * (64 / LPR);
    const int mid = min(r.count, (r.count / 2 + kChunk - 1) / kChunk * kChunk);
    if (pair_half) pp0 = mid;
    else pp1 = mid;
  }
  if (kPair) {
    topk::criticality_scan_head<T, LPR, G, kHeadThreads, UC, true, true>(
        (const T*)a.q, a.qsb, a.qsh, (const T*)t.kmin, (const T*)t.kmax, t.ssb, t.ssh, t.ssp,
        a.slopes, (T*)t.scores, a.H, t.num_pages, pp1, a.page_size, r.seq_len, r.q_pos, b, kvh,
        G == 1 ? keys : head_keys, G == 1 ? &sel_hist[0][0] : nullptr, &scan_next,
        t.scan_rev != 0, t.scan_nt != 0, pp0);
    __builtin_amdgcn_s_waitcnt(0);  // the stores through are complete
  } else if (!t.prescored) {
    topk::criticality_scan_head<T, LPR, G, kHeadThreads, UC, true>(
        (const T*)a.q, a.qsb, a.qsh, (const T*)t.kmin, (const T*)t.kmax, t.ssb, t.ssh, t.ssp,
        a.slopes, (T*)t.scores, a.H, t.num_pages, r.count, a.page_size, r.seq_len, r.q_pos, b,
        kvh, G == 1 ? (keep ? keys : nullptr) : head_keys,
        G == 1 && keep ? &sel_hist[0][0] : nullptr, &scan_next, t.scan_rev != 0,
        t.scan_nt != 0);
  } else if (G > 1 && head_keys &&
             (t.num_pages * (int)sizeof(T)) % 16 == 0 && ((uintptr_t)sbase & 15) == 0) {
    // every query head's keys into LDS once (the select reads them per pass):
    // 16-byte loads (each head's row of scores is 16-byte aligned, and the
    // last vector of a row stays within it), four per thread in flight
    constexpr int E = 16 / sizeof(T);
    const int per_row = (r.count + E - 1) / E;
    const int total = G * per_row;
    for (int i0 = 0; i0 < total; i0 += 4 * kHeadThreads) {
      uint4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = min(i0 + j * kHeadThreads + (int)threadIdx.x, total - 1);
        v[j] = ld16(sbase + (int64_t)(i / per_row) * t.num_pages + (i % per_row) * E);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = i0 + j * kHeadThreads + (int)threadIdx.x;
        if (i < total) {
          const int g = i / per_row, p0 = (i % per_row) * E;
          T x[E];
          __builtin_memcpy(x, &v[j], 16);
#pragma unroll
          for (int e = 0; e < E; ++e)
            if (p0 + e < r.count) head_keys[g * t.num_pages + p0 + e] = topk::ScoreKey<T>::key(x[e]);
        }
      }
    }
  } else if (G > 1 && head_keys) {
    // unaligned rows: element loads, eight per thread in flight
    const int total = G * r.count;
    for (int i0 = 0; i0 < total; i0 += 8 * kHeadThreads) {
      T sv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = min(i0 + j * kHeadThreads + (int)threadIdx.x, total - 1);
        sv[j] = sbase[(i / r.count) * t.num_pages + i % r.count];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = i0 + j * kHeadThreads + (int)threadIdx.x;
        if (i < total) head_keys[(i / r.count) * t.num_pages + i % r.count] = topk::ScoreKey<T>::key(sv[j]);
      }
    }
  }
  __syncthreads();
  if constexpr (kPair) {
    if (threadIdx.x == 0) {
      const unsigned long long old = __hip_atomic_exchange(
          t.pair_cnt + bkv, t.pair_tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool second = old == t.pair_tag;
      if (second)
        __hip_atomic_store(t.pair_cnt + bkv, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      scan_next = second ? 1 : 0;
    }
    __syncthreads();
    if (scan_next == 0) return;  // the partner selects and decodes
    // the partner's half: its scores' keys (G == 1: and first-digit counts;
    // G > 1: every query head's keys)
    const int q0 = pair_half ? 0 : pp1, q1 = pair_half ? pp0 : r.count;
    if constexpr (G == 1) {
      for (int p = q0 + (int)threadIdx.x; p < q1; p += kHeadThreads) {
        const uint32_t key = topk::ScoreKey<T>::key(topk::load_through(sbase + p));
        keys[p] = key;
        atomicAdd(&sel_hist[0][key >> (topk::ScoreKey<T>::kBits - 8)], 1u);
      }
    } else {
      const int w = q1 - q0;
      for (int i = (int)threadIdx.x; i < G * w; i += kHeadThreads) {
        const int g = i / w, p = q0 + i % w;
        head_keys[g * t.num_pages + p] =
            topk::ScoreKey<T>::key(topk::load_through(sbase + (int64_t)g * t.num_pages + p));
      }
    }
    __syncthreads();
  }
  EKV_STAMP(1);
  int32_t* pi = const_cast<int32_t*>(a.page_indices) + b * a.pisb + kvh * a.pish;
  // G == 1: the scan left the keys in LDS; prescored, the select stages them
  const bool staged = kPair || (keep && !t.prescored);
  // the page table goes to LDS only here and to global memory at the end, so
  // that no barrier of the select or the decode waits on its stores
  topk::topk_select_block<T, G, kHeadThreads>(
      sbase, t.num_pages, r.count, r.k, r.last_page, nullptr, keys, keep ? r.count : 0, staged,
      s_pages, list, head_keys, t.num_pages, t.list_words, G == 1 ? sel_hist : nullptr,
      G == 1 && staged);
  EKV_WSTAMP(4);
  __syncthreads();
  EKV_STAMP(2);
  const int n = token_count(a, b, kvh);
  decode_head_body<T, LPR, G, UD, true, true>(a, b, kvh, n, stage, a.stage_cap, sh);
  const int slots = min(r.k, r.count) + (r.last_page >= 0 ? 1 : 0);
  for (int i = threadIdx.x; i < slots; i += kHeadThreads) pi[i] = s_pages[i];
}

// Gaussian selection of one step, as read by the fused kernel (see
// ekv_gaussian_paged_entmax_decode).
struct GaussArgs {
  gauss::SelectArgs sel;
  const float4* partials;  // [B, H, splits] from the moments launch
  int splits;
  float* mu_g;             // [B, H] outputs
  float* sigma_g;
  float* mean_var;
  float* var_means;
  float* tau_hat;          // [B, H] tau-hat out (in when tau_hat_given)
  int tau_hat_given;       // tau-hat precomputed (page mixture)
  float tau_alpha;
  float n_tokens, log_n_factor;
  int tau_iters;
  float tol;
  // the paired launch (groups of 4 and 8 at most half the CU count): two
  // workgroups per (b, kv head) share the K scoring of selections of at least
  // kPairMinTokens tokens (below that the second leaves after the
  // selection); one arrival word per pair (see pair_handoff)
  unsigned long long* pair_cnt = nullptr;
  unsigned long long pair_tag = 0;
};

constexpr int kPairMinTokens = 8192;

// One (b, kv head) per workgroup end to end: the global moments of every head
// (for the batch-wide mean sigma_g of the automatic margins) and of its own G
// heads, their tau-hat (one wave per head), threshold selection + pack +
// clamp, then phases 1-3 of the decode on the selected pages starting from
// the clamped tau (given-tau mode) or solving it (exact mode).
template <typename T, int LPR, int G, int UD, bool kPair = false>
__global__ __launch_bounds__(kHeadThreads) void gaussian_decode_kernel(DecodeArgs a, GaussArgs f) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int D = LPR * VEC;
  extern __shared__ __attribute__((aligned(16))) float stage[];
  __shared__ __attribute__((aligned(16))) int hist[kWaves][kBins];
  __shared__ float4 part[2 * kWaves];
  __shared__ float s_tau[G];
  __shared__ int sup_row[sup_chunk(G)];
  __shared__ float sup_p[G * sup_chunk(G)];
  __shared__ int flag_cnt[kWaves];
  __shared__ float red[kWaves * D];
  __shared__ int s_pages[kTablePages];
  __shared__ float s_th[G], s_sg[G], s_tin[G];
  __shared__ float scratch[kWaves];
  __shared__ float ups[G][kWaves];
  __shared__ float wmax[G * kWaves];
  HeadShared sh{hist, part, s_tau, sup_row, sup_p, flag_cnt, red, s_pages};
  sh.tau_in_lds = s_tin;
  sh.wmax = wmax;

  const int tid = threadIdx.x, wid = tid >> 6;
  const int bkv = kPair ? blockIdx.x >> 1 : blockIdx.x;
  const int pair_half = kPair ? blockIdx.x & 1 : 0;
  const int b = bkv / a.Hkv, kvh = bkv % a.Hkv;
  const gauss::SelectArgs& sel = f.sel;
  EKV_STAMP(0);
  // Global moments from the moments launch's partials, reduced over aligned
  // groups of S2 lanes (one fixed lane-tree, so every consumer derives the same
  // bits).  Wave g < G reduces its own head and solves its tau-hat while the
  // other waves reduce every head of the batch for the mean sigma_g of the
  // automatic margins.
  const int nh = sel.B * sel.H;
  const int s2 = gauss::split_lanes(f.splits);
  const int own0 = b * a.H + kvh * G;
  const int lane = tid & 63;
  // this sequence's statistics pages (ragged batch) within rows of stride sel.pages
  const int own_pages = sel.seq_lens
                            ? min(seq_pages(sel.seq_lens[b], sel.page_size).stat_pages, sel.pages)
                            : sel.pages;
  if (wid < G) {
    const int h = own0 + wid;
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (lane < f.splits) x = f.partials[(int64_t)h * f.splits + lane];
    if (lane >= s2) x = make_float4(0.f, 0.f, 0.f, 0.f);
    x = gauss::reduce_splits(x, s2);
    x.x = __shfl(x.x, 0);
    x.y = __shfl(x.y, 0);
    x.z = __shfl(x.z, 0);
    const gauss::TauGeom tg = gauss::tau_geom(sel.seq_lens, b, sel.page_size, sel.pages,
                                              f.n_tokens, f.log_n_factor);
    const gauss::Moments m = gauss::finalize_moments(x, tg.pages);
    EKV_STAMP(7);
    const float th = f.tau_hat_given
                         ? f.tau_hat[h]
                         : gauss::solve_single_gaussian_wave(m.mu_g, m.sigma_g, tg.n,
                                                             f.tau_alpha, tg.lnf, f.tau_iters,
                                                             f.tol);
    if (lane == 0) {
      s_th[wid] = th;
      s_sg[wid] = m.sigma_g;
      f.mu_g[h] = m.mu_g;
      f.sigma_g[h] = m.sigma_g;
      f.mean_var[h] = m.mean_var;
      f.var_means[h] = m.var_means;
      if (!f.tau_hat_given) f.tau_hat[h] = th;
    }
  } else {
    const int nt = (kWaves - G) * 64, t = tid - G * 64;
    if (sel.auto_margins) {
      const int hpp = nt / s2;  // heads per pass
      float ssum = 0.f;
      for (int base = 0; base < nh; base += hpp) {
        const int h = base + t / s2, j = t % s2;
        const bool ok = t < hpp * s2 && h < nh;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ok && j < f.splits) x = f.partials[(int64_t)h * f.splits + j];
        x = gauss::reduce_splits(x, s2);
        if (ok && j == 0) {
          const int hp = sel.seq_lens ? seq_pages(sel.seq_lens[h / a.H], sel.page_size).stat_pages
                                      : sel.pages;
          ssum += gauss::finalize_moments(x, hp).sigma_g;
        }
      }
      ssum = wave_sum(ssum);
      if (lane == 0) scratch[wid] = ssum;
    }
    // the selection's mean of mu_p + 1.5 sigma_p per head (independent of tau-hat)
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int64_t row = ((int64_t)b * a.H + kvh * G + g) * sel.pages;
      float u = 0.f;
      for (int p = t; p < own_pages; p += nt)
        u += fma_rn(1.5f, sel.sigma_p[row + p], sel.mu_p[row + p]);
      u = wave_sum(u);
      if (lane == 0) ups[g][wid] = u;
    }
  }
  __syncthreads();
  float sbar = 0.f;
  if (sel.auto_margins) {
    for (int w = G; w < kWaves; ++w) sbar += scratch[w];
    sbar /= (float)nh;
  }
  // every thread forms the means itself (same order, same bits): no second barrier
  float upper[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float u = 0.f;
    for (int w = G; w < kWaves; ++w) u += ups[g][w];
    upper[g] = u / (float)own_pages;
  }
  EKV_STAMP(6);
  EKV_STAMP(1);
  const int count = gauss::select_pack_block<G, kHeadThreads>(sel, b, kvh, sbar, s_th, s_sg,
                                                              s_pages, kTablePages, s_tin,
                                                              upper);
  __syncthreads();
  EKV_STAMP(2);

  // compacted length max(count - 1, 0) * ps + last_page_size; an empty table
  // attends to nothing
  const int lps = sel.seq_lens ? seq_pages(sel.seq_lens[b], sel.page_size).last_size
                               : sel.last_page_size;
  int n = count > 0 ? (count - 1) * sel.page_size + lps : 0;
  n = min(n, min(count * sel.page_size, a.max_tokens));
  // paired: both workgroups selected the same pages (and stored the same
  // outputs); they share the scoring of large selections, and the second
  // leaves at once for small ones
  unsigned long long* word = nullptr;
  if constexpr (kPair) {
    if (n < kPairMinTokens && pair_half) return;
    if (n >= kPairMinTokens) word = f.pair_cnt + bkv;
  }
  // the first kTablePages page ids are already in s_pages (all of them when
  // count <= kTablePages: the decode then reads no page id from global memory)
  if (n <= a.stage_cap && count <= kTablePages) {
    decode_head_body<T, LPR, G, UD, true, true>(a, b, kvh, n, stage, a.stage_cap, sh, false,
                                                word, f.pair_tag, pair_half);
  } else if (n <= a.stage_cap) {
    decode_head_body<T, LPR, G, UD, true>(a, b, kvh, n, stage, a.stage_cap, sh, true, word,
                                          f.pair_tag, pair_half);
  } else {
    float* ws = a.ws_scores + ((int64_t)b * a.H + kvh * G) * a.max_tokens;
    decode_head_body<T, LPR, G, UD, false>(a, b, kvh, n, ws, a.max_tokens, sh, true, word,
                                           f.pair_tag, pair_half);
  }
}

constexpr int kStageBytes = 96 * 1024;


// Host launchers of one storage type T and GQA group G, explicitly
// instantiated per (T, G) in decode_inst.hip (one object per pair, so the
// kernels compile in parallel) and called by the C entry points.
template <typename T, int G>
struct Launch {
  // split scoring (when !head_path) + decode_head_kernel
  static int decode(DecodeArgs a, int B, int Hkv, int D, bool head_path, hipStream_t s);
  // the fused criticality + top-k + decode launch; *handled = 0 when the
  // shape does not fit one workgroup's LDS (the caller then runs two launches)
  static int topk(DecodeArgs a, SelectArgs t, int B, int Hkv, int D, int tokens, hipStream_t s,
                  int* handled);
  // the fused Gaussian select + decode launch
  static int gaussian(DecodeArgs a, GaussArgs f, int B, int Hkv, int D, int max_tokens,
                      hipStream_t s);
};

}  // namespace dec
}  // namespace ekv
