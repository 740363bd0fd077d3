// batch_topk for AMD Instinct MI355X (gfx950) -- C++ drop-in for the reference host API.
//
// Same namespace, names and argument order as the reference's include/batch_topk.cuh:10-21,
// spelled with HIP types (__half, hipError_t, hipStream_t).  A C++ caller of
// radix_topk::batch_topk_half recompiles against this header unchanged apart from those
// type names.  Every function forwards to the C ABI in batch_topk.h; none adds a symbol
// to the shared library.
#ifndef BATCH_TOPK_AMD_BATCH_TOPK_HPP_
#define BATCH_TOPK_AMD_BATCH_TOPK_HPP_

#include <cstddef>
#include <cstdint>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include "batch_topk.h"

// The bf16 entry points take pointers only, so the type is declared here rather than taken
// from <hip/hip_bf16.h> (which needs a compiler with a native bf16 type); a caller that
// includes that header gets the same struct.
struct __hip_bfloat16;

namespace radix_topk {

inline constexpr int kMaxSupportedK = RADIX_TOPK_MAX_K;

// Reference include/batch_topk.cuh:10-19.
inline hipError_t batch_topk_half(const __half* d_input, int seg_num, int seg_len, int k,
                                  __half* d_output_values, int* d_output_indices,
                                  void* d_workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
  return static_cast<hipError_t>(radix_topk_batch_topk_half(
      reinterpret_cast<const uint16_t*>(d_input), seg_num, seg_len, k,
      reinterpret_cast<uint16_t*>(d_output_values), reinterpret_cast<int32_t*>(d_output_indices),
      d_workspace, workspace_bytes, reinterpret_cast<void*>(stream)));
}

// Reference include/batch_topk.cuh:21.
inline size_t batch_topk_half_workspace_size(int seg_num, int seg_len, int k) {
  return radix_topk_batch_topk_half_workspace_size(seg_num, seg_len, k);
}

// Segmented extension (no reference counterpart): offsets are a device int32 array.
inline hipError_t batch_topk_half_segmented(const __half* d_input, const int32_t* d_offsets,
                                            int seg_num, int max_seg_len, int k,
                                            __half* d_output_values, int* d_output_indices,
                                            void* d_workspace, size_t workspace_bytes,
                                            hipStream_t stream) {
  return static_cast<hipError_t>(radix_topk_batch_topk_half_segmented(
      reinterpret_cast<const uint16_t*>(d_input), d_offsets, seg_num, max_seg_len, k,
      reinterpret_cast<uint16_t*>(d_output_values), reinterpret_cast<int32_t*>(d_output_indices),
      d_workspace, workspace_bytes, reinterpret_cast<void*>(stream)));
}

inline size_t batch_topk_half_segmented_workspace_size(int seg_num, int max_seg_len, int k) {
  return radix_topk_batch_topk_half_segmented_workspace_size(seg_num, max_seg_len, k);
}

// bfloat16 twins (no reference counterpart; see batch_topk.h).
inline hipError_t batch_topk_bf16(const __hip_bfloat16* d_input, int seg_num, int seg_len, int k,
                                  __hip_bfloat16* d_output_values, int* d_output_indices,
                                  void* d_workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
  return static_cast<hipError_t>(radix_topk_batch_topk_bf16(
      reinterpret_cast<const uint16_t*>(d_input), seg_num, seg_len, k,
      reinterpret_cast<uint16_t*>(d_output_values), reinterpret_cast<int32_t*>(d_output_indices),
      d_workspace, workspace_bytes, reinterpret_cast<void*>(stream)));
}

inline size_t batch_topk_bf16_workspace_size(int seg_num, int seg_len, int k) {
  return radix_topk_batch_topk_bf16_workspace_size(seg_num, seg_len, k);
}

inline hipError_t batch_topk_bf16_segmented(const __hip_bfloat16* d_input, const int32_t* d_offsets,
                                            int seg_num, int max_seg_len, int k,
                                            __hip_bfloat16* d_output_values, int* d_output_indices,
                                            void* d_workspace, size_t workspace_bytes,
                                            hipStream_t stream) {
  return static_cast<hipError_t>(radix_topk_batch_topk_bf16_segmented(
      reinterpret_cast<const uint16_t*>(d_input), d_offsets, seg_num, max_seg_len, k,
      reinterpret_cast<uint16_t*>(d_output_values), reinterpret_cast<int32_t*>(d_output_indices),
      d_workspace, workspace_bytes, reinterpret_cast<void*>(stream)));
}

inline size_t batch_topk_bf16_segmented_workspace_size(int seg_num, int max_seg_len, int k) {
  return radix_topk_batch_topk_bf16_segmented_workspace_size(seg_num, max_seg_len, k);
}

}  // namespace radix_topk

#endif  // BATCH_TOPK_AMD_BATCH_TOPK_HPP_
