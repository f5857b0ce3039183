// The top-k decode step for callers that cannot allocate device memory (code
// under graph capture, serving loops that forbid hipMalloc): the step's
// workspace is a file-scope device array instead of a caller buffer.
//
// ekv_topk_paged_entmax_decode needs a workspace only for the fp32 scores of
// heads that are scored outside the fused launch (B * Hkv below the fused
// threshold, ragged batches, or token lists that do not fit LDS); it needs no
// initialisation, so nothing is cleared here.  Every call on one GPU shares
// that GPU's array: calls that overlap on one GPU (two streams, two host
// threads) race on it and must be serialised by the caller.
#include <atomic>

#include "ekv_common.h"
#include "../../include/entmaxkv.h"

using namespace ekv;

namespace {

constexpr int64_t kScratchBytes = EKV_NOALLOC_SCRATCH_BYTES;  // include/entmaxkv.h
constexpr int kMaxDevices = 64;

// One copy per GPU, held until the process ends.  In host code this name is a
// stand-in, not a device address: only the pointer from hipGetSymbolAddress
// below is ever handed to a kernel.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::atomic<void*> g_scratch_ptr[kMaxDevices];

// The device address of this GPU's copy of `scratch`, looked up once per
// device with that device current (the caller's current device).
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(EKV_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(EKV_ERR_ARG, "device %d beyond the %d supported", dev, kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(EKV_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return EKV_OK;
}

}  // namespace

extern "C" int ekv_topk_paged_entmax_decode_noalloc(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kmin, const void* kmax,
    int64_t s_stride_b, int64_t s_stride_h, int64_t s_stride_page, void* scores, int num_pages,
    int seq_len, int q_pos, int k_select, int last_page, const void* k, const void* v,
    int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_row, int64_t kv_rows,
    const int32_t* block_table, int64_t bt_stride_b, int bt_blocks,
    int32_t* page_indices, int64_t pi_stride_b, int64_t pi_stride_h,
    const int32_t* cache_seqlens, int64_t cs_stride_b, int64_t cs_stride_h,
    const int32_t* q_seqlens, const float* alibi_slopes, const int32_t* seq_lens, float* tau,
    int niter, void* out, int64_t out_stride_b, int64_t out_stride_h, float alpha, float qscale,
    int page_size, int B, int H, int Hkv, int D, int splits, int max_tokens, int dtype,
    void* stream) {
  EKV_REQUIRE(B > 0 && H > 0 && max_tokens > 0,
              "ekv_topk_paged_entmax_decode_noalloc: bad sizes");
  const int64_t need = ekv_decode_workspace_bytes(B, H, Hkv, D, splits, max_tokens);
  EKV_REQUIRE(need <= kScratchBytes,
              "ekv_topk_paged_entmax_decode_noalloc: the step needs %lld workspace bytes "
              "(ekv_decode_workspace_bytes), more than the %lld of the static scratch; use "
              "ekv_topk_paged_entmax_decode with a caller workspace",
              (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  return ekv_topk_paged_entmax_decode(
      q, q_stride_b, q_stride_h, kmin, kmax, s_stride_b, s_stride_h, s_stride_page, scores,
      num_pages, seq_len, q_pos, k_select, last_page, k, v, kv_stride_b, kv_stride_h,
      kv_stride_row, kv_rows, block_table, bt_stride_b, bt_blocks, page_indices, pi_stride_b, pi_stride_h, cache_seqlens, cs_stride_b,
      cs_stride_h, q_seqlens, alibi_slopes, seq_lens, tau, niter, out, out_stride_b, out_stride_h,
      alpha, qscale, page_size, B, H, Hkv, D, splits, max_tokens, ws, kScratchBytes, dtype,
      stream);
}
