// Allocation-free entry point: radix_topk_batch_topk_half with its workspace in a static
// device array instead of caller memory (include/batch_topk.h, radix_topk_batch_topk_half_noalloc).
//
// The array is one per GPU, allocated with the code object (so it lives until the process
// ends), and is shared by every call on that GPU: calls that overlap on one GPU race on it.
// Its device address is looked up once per device with hipGetSymbolAddress (the array's name
// is a host-side stand-in in host code) and the call then runs the plain entry point with it.
// The engine's workspace needs no initialisation (its content on entry may be arbitrary), so
// nothing is cleared between calls.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>

#include "../../include/batch_topk.h"

static constexpr size_t kScratchBytes = RADIX_TOPK_NOALLOC_SCRATCH_BYTES;

// The workspace of every allocation-free call on a GPU (file scope: one per GPU).
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// The current device's address of `scratch`, looked up on the first call on that device.
hipError_t scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return hipSuccess;
}

}  // namespace

extern "C" int radix_topk_batch_topk_half_noalloc(const uint16_t* d_input, int seg_num, int seg_len, int k,
                                                  uint16_t* d_output_values, int32_t* d_output_indices,
                                                  void* stream) {
  // Validation before any HIP call, as the plain entry point does it.
  const size_t need = radix_topk_batch_topk_half_workspace_size(seg_num, seg_len, k);
  if (need == 0 || !d_input || !d_output_values || !d_output_indices) return static_cast<int>(hipErrorInvalidValue);
  if (need > kScratchBytes) return static_cast<int>(hipErrorOutOfMemory);
  void* ws = nullptr;
  const hipError_t e = scratch_address(&ws);
  if (e != hipSuccess) return static_cast<int>(e);
  return radix_topk_batch_topk_half(d_input, seg_num, seg_len, k, d_output_values, d_output_indices, ws,
                                    kScratchBytes, stream);
}
