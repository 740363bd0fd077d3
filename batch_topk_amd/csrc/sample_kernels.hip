// Stand-alone top-k sampling kernel: one wave per row over the top-k rows the cooperative
// top-k grid wrote to global memory (every other plan samples inside the top-k kernel).  The
// rule is sample_ranked_row's (sample_row.hpp).

#include <hip/hip_runtime.h>

#include <cstdint>

#include "sample_row.hpp"
#include "topk_common.hpp"

namespace radix_topk_amd {
namespace {

__global__ void __launch_bounds__(64) topk_sample_kernel(SampleParams p) {
  const int row = blockIdx.x;
  const int k = p.k;
  const uint16_t* vals = p.topk_vals + static_cast<int64_t>(row) * k;
  const int32_t* idx = p.topk_idx + static_cast<int64_t>(row) * k;
  const bool bf16 = p.bf16 != 0;
  // Ranks with an index are a prefix of the row (pads follow): m = their count.
  int m_lane = 0;
  for (int r = threadIdx.x; r < k; r += 64) m_lane += idx[r] >= 0 ? 1 : 0;
  int m = m_lane;
  for (int off = 32; off > 0; off >>= 1) m += __shfl_xor(m, off, 64);
  auto get = [&](int r) { return RankedEntry{bits16_to_float(vals[r], bf16), idx[r]}; };
  sample_ranked_row(get, m, k, p.inv_temperature, p.uniforms[row], p.samples + row,
                    p.probs ? p.probs + static_cast<int64_t>(row) * k : nullptr);
}

}  // namespace

int launch_topk_sample(const SampleParams& params, void* stream) {
  hipLaunchKernelGGL(topk_sample_kernel, dim3(static_cast<unsigned>(params.seg_num)), dim3(64), 0,
                     static_cast<hipStream_t>(stream), params);
  return static_cast<int>(hipGetLastError());
}

}  // namespace radix_topk_amd
