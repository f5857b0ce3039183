// Shared device helpers for the EntmaxKV CDNA4 (gfx950) kernels.
//
// Conventions used by every kernel in this library:
//   * wave64; a "row segment" is the group of LPR consecutive lanes that hold
//     one D-long row, each lane owning VEC = 16 / sizeof(T) contiguous elements
//     (one 16-byte global load).  LPR = D / VEC is a power of two <= 64.
//   * arithmetic is fp32; storage types are fp32, fp16 or bf16.
//   * no kernel waits for another workgroup: results that need several
//     workgroups are combined by the next launch.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <climits>

#include <type_traits>

namespace ekv {

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

// ---------------------------------------------------------------------------
// storage types
// ---------------------------------------------------------------------------

struct bf16_t { uint16_t bits; };

template <typename T> struct Cvt;

template <> struct Cvt<float> {
  static __device__ __forceinline__ float to_f(float x) { return x; }
  static __device__ __forceinline__ float from_f(float x) { return x; }
};

template <> struct Cvt<_Float16> {
  static __device__ __forceinline__ float to_f(_Float16 x) { return (float)x; }
  static __device__ __forceinline__ _Float16 from_f(float x) { return (_Float16)x; }
};

template <> struct Cvt<bf16_t> {
  static __device__ __forceinline__ float to_f(bf16_t x) {
    return __uint_as_float(((uint32_t)x.bits) << 16);
  }
  // round to nearest even; NaN stays a quiet NaN
  static __device__ __forceinline__ bf16_t from_f(float x) {
    uint32_t u = __float_as_uint(x);
    bf16_t r;
    if ((u & 0x7fffffffu) > 0x7f800000u) {
      r.bits = (uint16_t)((u >> 16) | 0x40u);
    } else {
      u += 0x7fffu + ((u >> 16) & 1u);
      r.bits = (uint16_t)(u >> 16);
    }
    return r;
  }
};

template <typename T> __device__ __forceinline__ float to_f(T x) { return Cvt<T>::to_f(x); }
template <typename T> __device__ __forceinline__ T from_f(float x) { return Cvt<T>::from_f(x); }

// One 16-byte vector of T, converted to fp32 lanes.
template <typename T> struct Vec {
  static constexpr int N = 16 / sizeof(T);
  float v[N];
  __device__ __forceinline__ void load(const T* p) {
    uint4 raw = *reinterpret_cast<const uint4*>(p);
    const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = to_f<T>(e[i]);
  }
  __device__ __forceinline__ void store(T* p) const {
    uint4 raw;
    T* e = reinterpret_cast<T*>(&raw);
#pragma unroll
    for (int i = 0; i < N; ++i) e[i] = from_f<T>(v[i]);
    *reinterpret_cast<uint4*>(p) = raw;
  }
};

template <typename T> struct VecRaw {
  static constexpr int N = 16 / sizeof(T);
  uint4 raw;
  __device__ __forceinline__ void load(const T* p) { raw = *reinterpret_cast<const uint4*>(p); }
  // non-temporal when nt (see ld16_nt)
  __device__ __forceinline__ void load_sel(const T* p, bool nt) {
    if (nt) {
      typedef unsigned int u4 __attribute__((ext_vector_type(4)));
      const u4 v = __builtin_nontemporal_load(reinterpret_cast<const u4*>(p));
      raw = make_uint4(v.x, v.y, v.z, v.w);
    } else {
      raw = *reinterpret_cast<const uint4*>(p);
    }
  }
  __device__ __forceinline__ float get(int i) const {
    return to_f<T>(reinterpret_cast<const T*>(&raw)[i]);
  }
};

// ---------------------------------------------------------------------------
// 16-byte dot products in the storage format (exact 16-bit products,
// fp32 accumulation: v_dot2_f32_f16 / v_dot2_f32_bf16; fp32 uses fma)
// ---------------------------------------------------------------------------

typedef _Float16 ekv_half2 __attribute__((ext_vector_type(2)));
typedef short ekv_short2 __attribute__((ext_vector_type(2)));

template <typename T> struct Dot16;
template <> struct Dot16<_Float16> {
  static __device__ __forceinline__ float dot(const uint4& a, const uint4& b, float acc) {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(ekv_half2, a.x), __builtin_bit_cast(ekv_half2, b.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(ekv_half2, a.y), __builtin_bit_cast(ekv_half2, b.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(ekv_half2, a.z), __builtin_bit_cast(ekv_half2, b.z), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(ekv_half2, a.w), __builtin_bit_cast(ekv_half2, b.w), acc, false);
    return acc;
  }
  // per-element all-ones mask where the element is >= 0 (+0.0 and -0.0 included)
  static __device__ __forceinline__ uint4 nonneg_mask(const uint4& q) {
    auto m = [](uint32_t w) {
      const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
      const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
      return ((float)lo >= 0.f ? 0x0000ffffu : 0u) | ((float)hi >= 0.f ? 0xffff0000u : 0u);
    };
    return make_uint4(m(q.x), m(q.y), m(q.z), m(q.w));
  }
};
template <> struct Dot16<bf16_t> {
  static __device__ __forceinline__ float dot(const uint4& a, const uint4& b, float acc) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ekv_short2, a.x), __builtin_bit_cast(ekv_short2, b.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ekv_short2, a.y), __builtin_bit_cast(ekv_short2, b.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ekv_short2, a.z), __builtin_bit_cast(ekv_short2, b.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(ekv_short2, a.w), __builtin_bit_cast(ekv_short2, b.w), acc, false);
    return acc;
  }
  static __device__ __forceinline__ uint4 nonneg_mask(const uint4& q) {
    auto m = [](uint32_t w) {
      const float lo = __uint_as_float(w << 16);
      const float hi = __uint_as_float(w & 0xffff0000u);
      return (lo >= 0.f ? 0x0000ffffu : 0u) | (hi >= 0.f ? 0xffff0000u : 0u);
    };
    return make_uint4(m(q.x), m(q.y), m(q.z), m(q.w));
  }
};
template <> struct Dot16<float> {
  static __device__ __forceinline__ float dot(const uint4& a, const uint4& b, float acc) {
    acc = fmaf(__uint_as_float(a.x), __uint_as_float(b.x), acc);
    acc = fmaf(__uint_as_float(a.y), __uint_as_float(b.y), acc);
    acc = fmaf(__uint_as_float(a.z), __uint_as_float(b.z), acc);
    acc = fmaf(__uint_as_float(a.w), __uint_as_float(b.w), acc);
    return acc;
  }
  static __device__ __forceinline__ uint4 nonneg_mask(const uint4& q) {
    auto m = [](uint32_t w) { return __uint_as_float(w) >= 0.f ? 0xffffffffu : 0u; };
    return make_uint4(m(q.x), m(q.y), m(q.z), m(q.w));
  }
};

// Element-wise (mask ? b : a) on 16-byte vectors (v_bfi_b32).
__device__ __forceinline__ uint4 bit_select(const uint4& a, const uint4& b, const uint4& mask) {
  return make_uint4((b.x & mask.x) | (a.x & ~mask.x), (b.y & mask.y) | (a.y & ~mask.y),
                    (b.z & mask.z) | (a.z & ~mask.z), (b.w & mask.w) | (a.w & ~mask.w));
}

__device__ __forceinline__ uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }
// A non-temporal 16-byte load (`nt`): for data streamed once per step (the
// page statistics of the scans), so that it does not push out of the caches
// what the step reads again (K and V rows).
__device__ __forceinline__ uint4 ld16_nt(const void* p) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  const u4 v = __builtin_nontemporal_load(reinterpret_cast<const u4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ld16_sel(const void* p, bool nt) {
  return nt ? ld16_nt(p) : ld16(p);
}

// Statistics scans stream their bounds / moments with non-temporal loads when
// they read more than this per launch: beyond it they cannot stay in the
// GPU's 256 MB memory-side cache from one step to the next anyway, and
// normal loads would push out the K and V rows that the next step reads
// again; below it (128 MiB at B4 H32 L32k) normal loads keep them cached.
constexpr int64_t kStreamNtBytes = 160ll << 20;

// Whether a scan of two [B, Hkv, pages, D] statistics of storage dtype code
// `dtype` (0 fp32, 1 fp16, 2 bf16) streams with non-temporal loads.
inline bool stream_nt(int B, int Hkv, int pages, int D, int dtype) {
  const int64_t esize = dtype == 0 ? 4 : 2;
  return (int64_t)B * Hkv * pages * D * esize * 2 > kStreamNtBytes;
}

// ---------------------------------------------------------------------------
// wave-level reductions (wave64)
// ---------------------------------------------------------------------------

// Lane exchanges without the LDS crossbar: DPP within a row of 16 lanes and
// the gfx950 permlane swaps across rows (v_permlane16_swap_b32 exchanges the
// odd rows of one register with the even rows of another, v_permlane32_swap_b32
// the upper half with the lower half; applied to two copies of one value, the
// two results hold the value of lane i and of lane i ^ 16 (resp. ^ 32)).
namespace lanes {
// DPP controls (GCN/CDNA encoding)
constexpr int kQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;  // lane i <- 7 - i within 8
constexpr int kRowMirror = 0x140;      // lane i <- 15 - i within 16
constexpr int kRowRor4 = 0x124;        // lane i <- (i + 4) % 16 within 16
constexpr int kRowRor8 = 0x128;        // lane i <- (i + 8) % 16 within 16

template <int CTRL> __device__ __forceinline__ uint32_t dpp(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false);
}
// (value of lane i, value of lane i ^ 16)
__device__ __forceinline__ void swap16(uint32_t x, uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  a = r[0];
  b = r[1];
}
__device__ __forceinline__ void swap32(uint32_t x, uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  a = r[0];
  b = r[1];
}

struct Add {
  template <typename V> __device__ __forceinline__ V operator()(V a, V b) const { return a + b; }
};
struct Max {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
  __device__ __forceinline__ int operator()(int a, int b) const { return a > b ? a : b; }
};

template <typename V> __device__ __forceinline__ uint32_t bits(V x) {
  return __builtin_bit_cast(uint32_t, x);
}
template <typename V> __device__ __forceinline__ V from_bits(uint32_t x) {
  return __builtin_bit_cast(V, x);
}

// All-reduce over aligned segments of L lanes (L a power of two <= 64).
template <int L, typename V, typename Op>
__device__ __forceinline__ V seg_reduce(V x, Op op) {
  if constexpr (L >= 2) x = op(x, from_bits<V>(dpp<kQuadXor1>(bits(x))));
  if constexpr (L >= 4) x = op(x, from_bits<V>(dpp<kQuadXor2>(bits(x))));
  if constexpr (L >= 8) x = op(x, from_bits<V>(dpp<kRowHalfMirror>(bits(x))));
  if constexpr (L >= 16) x = op(x, from_bits<V>(dpp<kRowMirror>(bits(x))));
  if constexpr (L >= 32) {
    uint32_t a, b;
    swap16(bits(x), a, b);
    x = op(from_bits<V>(a), from_bits<V>(b));
  }
  if constexpr (L >= 64) {
    uint32_t a, b;
    swap32(bits(x), a, b);
    x = op(from_bits<V>(a), from_bits<V>(b));
  }
  return x;
}

// Sum over the lanes of a wave that share the same position within their
// segment of L lanes (lane i and every lane i ^ (m * L)); every lane receives
// the sum of its position.
template <int L>
__device__ __forceinline__ float cross_seg_sum(float x) {
  if constexpr (L <= 4) x += from_bits<float>(dpp<kRowRor8>(bits(x)));
  if constexpr (L <= 4) x += from_bits<float>(dpp<kRowRor4>(bits(x)));
  if constexpr (L == 8) x += from_bits<float>(dpp<kRowRor8>(bits(x)));
  if constexpr (L <= 16) {
    uint32_t a, b;
    swap16(bits(x), a, b);
    x = from_bits<float>(a) + from_bits<float>(b);
  }
  if constexpr (L <= 32) {
    uint32_t a, b;
    swap32(bits(x), a, b);
    x = from_bits<float>(a) + from_bits<float>(b);
  }
  return x;
}
}  // namespace lanes

// Sum over an aligned segment of L lanes (L a power of two <= 64); every lane
// of the segment receives the result.
template <int L> __device__ __forceinline__ float seg_sum(float x) {
  return lanes::seg_reduce<L>(x, lanes::Add{});
}

__device__ __forceinline__ float wave_sum(float x) { return seg_sum<64>(x); }

__device__ __forceinline__ float wave_max(float x) {
  return lanes::seg_reduce<64>(x, lanes::Max{});
}

__device__ __forceinline__ int wave_sum_i(int x) { return lanes::seg_reduce<64>(x, lanes::Add{}); }

// Inclusive prefix sum over the 64 lanes of a wave: Hillis-Steele steps
// within each row of 16 lanes (DPP row_shr), then the row totals carried
// across rows (DPP row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2
// and 3).  Lanes without a source read 0.
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return x;
}

// Block-wide exclusive scan of one int per thread (blockDim.x <= 1024).
// `scratch` must hold blockDim.x / 64 + 1 ints.  Returns the exclusive prefix;
// *total receives the block sum.  Contains __syncthreads.
__device__ __forceinline__ int block_excl_scan(int x, int* scratch, int* total) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nw = (blockDim.x + 63) >> 6;
  int inc = wave_incl_scan(x);
  if (lane == 63) scratch[wid] = inc;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < nw; ++w) {
      int c = scratch[w];
      scratch[w] = run;
      run += c;
    }
    scratch[nw] = run;
  }
  __syncthreads();
  int res = scratch[wid] + inc - x;
  *total = scratch[nw];
  __syncthreads();
  return res;
}

// Block-wide sum of a float (deterministic order).  `scratch` >= 16 floats.
__device__ __forceinline__ float block_sum(float x, float* scratch) {
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  const int nw = (blockDim.x + 63) >> 6;
  x = wave_sum(x);
  if (lane == 0) scratch[wid] = x;
  __syncthreads();
  float r = 0.f;
  for (int w = 0; w < nw; ++w) r += scratch[w];
  __syncthreads();
  return r;
}

// ---------------------------------------------------------------------------
// page geometry of one sequence
// ---------------------------------------------------------------------------

// A sequence of `len` tokens in pages of `ps`: `pages` including the partial
// last page; `stat_pages`, the pages the Gaussian statistics cover (all but
// the last when there are two or more, gaussian_utils.py:101-102,
// attention_gaussian.py:65-66); `stat_tokens`, the tokens of those pages
// (seq_len_for_stats); `last_size`, the last page's token count
// (attention_gaussian.py:79).  Top-k scores pages - 1 pages
// (attention_topk.py:49-50).  With a batch of ragged lengths every
// (b, kv head) workgroup derives its own geometry from seq_lens[b].
struct SeqPages {
  int pages, stat_pages, stat_tokens, last_size;
};
__host__ __device__ __forceinline__ SeqPages seq_pages(int len, int ps) {
  SeqPages g;
  g.pages = (len + ps - 1) / ps;
  g.stat_pages = g.pages > 1 ? g.pages - 1 : g.pages;
  g.stat_tokens = g.pages > 1 ? (g.pages - 1) * ps : len;
  g.last_size = g.pages > 0 ? len - (g.pages - 1) * ps : 0;
  return g;
}

// ---------------------------------------------------------------------------
// fp32 helpers with an explicit rounding sequence (no contraction)
// ---------------------------------------------------------------------------

__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ float sub_rn(float a, float b) { return __fsub_rn(a, b); }
__device__ __forceinline__ float fma_rn(float a, float b, float c) { return __fmaf_rn(a, b, c); }

}  // namespace ekv

// ---------------------------------------------------------------------------
// host-side error reporting shared by all entry points
// ---------------------------------------------------------------------------

#define EKV_OK 0
#define EKV_ERR_ARG (-1)
#define EKV_ERR_HIP (-2)

namespace ekv {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Compute units of the current device (queried once per device).
int device_cus();

// LDS one workgroup can allocate (gfx950).
constexpr int kLdsPerWorkgroup = 160 * 1024;
// The fused one-workgroup-per-(b, kv head) launches win when there are at
// least half as many heads as compute units: below that, a head's scan spread
// over many workgroups finishes sooner.  Measured at 128 heads on 256 CUs
// (benchmark configs 3 and 4) the fused launches are faster for the top-k step
// and for Gaussian selections of tens of pages, slower by 30 % for a
// Gaussian selection of half the cache.  Ragged batches always split: one
// workgroup per head would wait on the longest sequence.
inline bool one_workgroup_per_head(int heads, bool ragged) {
  return !ragged && 2 * heads >= device_cus();
}
}  // namespace ekv

namespace ekv {

// Runtime dtype code -> storage type T (passed as a value of type T).
// head_dim -> lanes per row (LPR) as an integral_constant.
template <typename T, typename F>
inline int dispatch_lpr(int D, F&& f) {
  constexpr int VEC = 16 / sizeof(T);
  if (D % VEC) return set_error(EKV_ERR_ARG, "head_dim %d must be a multiple of %d", D, VEC);
  switch (D / VEC) {
    case 4: return f(std::integral_constant<int, 4>{});
    case 8: return f(std::integral_constant<int, 8>{});
    case 16: return f(std::integral_constant<int, 16>{});
    case 32: return f(std::integral_constant<int, 32>{});
    case 64: return f(std::integral_constant<int, 64>{});
    default:
      return set_error(EKV_ERR_ARG, "head_dim %d unsupported (D/%d must be 4..64, power of two)", D,
                       VEC);
  }
}

template <typename F>
inline int dispatch_dtype(int dtype, F&& f) {
  switch (dtype) {
    case kF32: return f(float{});
    case kF16: return f(_Float16{});
    case kBF16: return f(bf16_t{});
    default: return set_error(EKV_ERR_ARG, "unknown dtype code %d", dtype);
  }
}

}  // namespace ekv

#define EKV_REQUIRE(cond, ...)                                  \
  do {                                                          \
    if (!(cond)) return ::ekv::set_error(EKV_ERR_ARG, __VA_ARGS__); \
  } while (0)
