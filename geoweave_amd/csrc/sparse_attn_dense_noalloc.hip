// gw_sparse_attn_fwd_dense_noalloc: the masked dense forward (gw_sparse_attn_fwd_dense) with
// its workspace in a fixed device array instead of caller memory, for callers that cannot
// allocate (HIP graph capture, serving loops). No counterpart in the reference.
#include <atomic>
#include <mutex>

#include "gw_common.h"

// ---------------------------------------------------------------------------------------
// Allocation-free variant: the workspace is a file-scope device array of a fixed size. It
// sits in this file alone, so in a code object of its own that HIP loads onto a device only
// when the array is first used there: a GPU holds its copy from this entry point's first call
// on it until the process ends, and processes that never call it hold none. Its device
// address is looked up on the first call on a device (hipGetSymbolAddress with that device
// current; a failed lookup is reported and tried again on the next call) and kept; host code
// never passes the array's name itself to a kernel. Every kernel of the call clears what it
// needs before use (selection words, flags, column maxima), so the array's contents from an
// earlier call do not matter; two calls that overlap on one GPU race on it.
// ---------------------------------------------------------------------------------------
namespace gw {
namespace {

constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
constexpr int kNoAllocMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::atomic<void*> g_scratch_ptr[kNoAllocMaxDevices];  // null until a lookup succeeded
std::mutex g_scratch_mu;

// The scratch array's address on the current device dev (looked up once it succeeds).
int scratch_address(int dev, void** out) {
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || ptr == nullptr) return hip_error(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                                              "hipGetSymbolAddress(scratch)");
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return GW_OK;
}

}  // namespace
}  // namespace gw

extern "C" size_t gw_sparse_attn_fwd_dense_noalloc_capacity(void) { return gw::kNoAllocScratchBytes; }

extern "C" int gw_sparse_attn_fwd_dense_noalloc(int dtype, const void* q, const int64_t* q_strides, const void* k,
                                                const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                                const int32_t* kv_pos, int64_t pos_stride_b, int64_t pos_stride_t,
                                                void* o, const int64_t* o_strides, float* lse, float* attn_sum,
                                                int64_t B, int64_t T, int64_t S, int64_t H, int64_t D, int64_t K,
                                                float softmax_scale, const void* logits, int logits_dtype,
                                                int64_t logits_stride_b, int64_t logits_stride_t, float eps,
                                                float* row_loss, void* stream) {
  using namespace gw;
  clear_error();
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_error(e, "hipGetDevice");
  if (dev < 0 || dev >= kNoAllocMaxDevices)
    return set_error(GW_ERR_UNSUPPORTED, "device %d is beyond the %d devices the allocation-free entry point serves",
                     dev, kNoAllocMaxDevices);
  void* scratch_ptr = nullptr;
  if (const int rc = scratch_address(dev, &scratch_ptr); rc != GW_OK) return rc;
  const size_t need = gw_sparse_attn_fwd_dense_workspace_size(B, T, S, H, D, K, attn_sum != nullptr ? 1 : 0);
  if (need > kNoAllocScratchBytes)
    return set_error(GW_ERR_UNSUPPORTED,
                     "this call needs %zu bytes of scratch; the allocation-free dense forward holds at most %zu "
                     "(use gw_sparse_attn_fwd_dense with a workspace)",
                     need, kNoAllocScratchBytes);
  return gw_sparse_attn_fwd_dense(dtype, q, q_strides, k, k_strides, v, v_strides, kv_pos, pos_stride_b, pos_stride_t,
                                  o, o_strides, lse, attn_sum, B, T, S, H, D, K, softmax_scale, logits, logits_dtype,
                                  logits_stride_b, logits_stride_t, eps, row_loss, scratch_ptr,
                                  kNoAllocScratchBytes, stream);
}
