// Top-k sampling over the rows the fused top-k kernel wrote (one wave per row).
//
// For a row whose top-k values in output order are v_0 >= v_1 >= ... (m = the number of
// ranks with an index >= 0, i.e. min(k, segment length)):
//   w_0 = 1;  for r >= 1: w_r = 1 if v_r == v_0, else exp((v_r - v_0) * inv_t), and 0 when
//   that is NaN (a NaN logit); a finite v_r below v_0 = +inf gets exp(-inf) = 0;
//   S = w_0 + ... + w_{m-1} (fp32);  the sample is the index at the first rank r whose
//   running sum w_0 + ... + w_r exceeds u * S (the last rank if rounding leaves none), and
//   probs[r] = w_r / S (0 for r >= m).  An empty row samples index -1.
// inv_t is 1 / temperature rounded to fp32 on the host.  Equal logits get equal weight,
// -inf logits weight 0 unless every rank is -inf (then they are equal to v_0).
//
// Each lane owns a contiguous run of ceil(k / 64) ranks: it computes their weights and its
// run's sum, a wave prefix sum gives every run its start, and the first lane whose run
// crosses u * S picks the rank inside its run.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "topk_common.hpp"

namespace radix_topk_amd {
namespace {

using u32 = uint32_t;
using u64 = unsigned long long;

constexpr int kMaxRun = (kMaxTopK + 63) / 64;  // ranks per lane at the largest k

__device__ __forceinline__ float bits_to_float(u32 b, bool bf16) {
  if (bf16) return __uint_as_float(b << 16);
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(b)));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, false));
}

// Inclusive prefix sum of one float per lane across a wave64 (DPP row shifts, then the row
// broadcasts carry row totals upward).
__device__ __forceinline__ float wave_scan_f(float x) {
  x += dpp_f<0x111, 0xf>(x);
  x += dpp_f<0x112, 0xf>(x);
  x += dpp_f<0x114, 0xf>(x);
  x += dpp_f<0x118, 0xf>(x);
  x += dpp_f<0x142, 0xa>(x);
  x += dpp_f<0x143, 0xc>(x);
  return x;
}

__device__ __forceinline__ int wave_scan_i(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);
  return x;
}

__global__ void __launch_bounds__(64) topk_sample_kernel(SampleParams p) {
  const int row = blockIdx.x;
  const int lane = threadIdx.x;
  const int k = p.k;
  const int run = (k + 63) / 64;
  const uint16_t* vals = p.topk_vals + static_cast<int64_t>(row) * k;
  const int32_t* idx = p.topk_idx + static_cast<int64_t>(row) * k;
  const bool bf16 = p.bf16 != 0;
  const float v0 = bits_to_float(vals[0], bf16);
  const int r0 = lane * run;

  float w[kMaxRun];
  float lane_sum = 0.0f;
  int m_lane = 0;  // valid ranks in this lane's run
#pragma unroll
  for (int t = 0; t < kMaxRun; ++t) {
    w[t] = 0.0f;
    const int r = r0 + t;
    if (t < run && r < k && idx[r] >= 0) {
      const float v = bits_to_float(vals[r], bf16);
      float x = (r == 0 || v == v0) ? 1.0f : expf((v - v0) * p.inv_temperature);
      if (x != x) x = 0.0f;
      w[t] = x;
      lane_sum += x;
      ++m_lane;
    }
  }
  const float incl = wave_scan_f(lane_sum);
  const float total = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(incl), 63));
  const int m = __builtin_amdgcn_readlane(wave_scan_i(m_lane), 63);  // min(k, length)
  if (m == 0) {
    if (lane == 0) p.samples[row] = -1;
    if (p.probs) {
      for (int r = lane; r < k; r += 64) p.probs[static_cast<int64_t>(row) * k + r] = 0.0f;
    }
    return;
  }
  const float target = p.uniforms[row] * total;
  // First rank of this lane's run whose running sum exceeds the target.
  float acc = incl - lane_sum;
  int hit = -1;
#pragma unroll
  for (int t = 0; t < kMaxRun; ++t) {
    if (t < run) {
      acc += w[t];
      if (hit < 0 && t < m_lane && acc > target) hit = r0 + t;
    }
  }
  const u64 lanes = __builtin_amdgcn_ballot_w64(hit >= 0);
  const int first = lanes ? static_cast<int>(__builtin_ctzll(lanes)) : -1;
  const int pick = first >= 0 ? __builtin_amdgcn_readlane(hit, first) : m - 1;
  if (lane == 0) p.samples[row] = idx[pick];
  if (p.probs) {
    const float inv_total = 1.0f / total;
    float* prow = p.probs + static_cast<int64_t>(row) * k;
#pragma unroll
    for (int t = 0; t < kMaxRun; ++t) {
      const int r = r0 + t;
      if (t < run && r < k) prow[r] = w[t] * inv_total;
    }
  }
}

}  // namespace

int launch_topk_sample(const SampleParams& params, void* stream) {
  hipLaunchKernelGGL(topk_sample_kernel, dim3(static_cast<unsigned>(params.seg_num)), dim3(64), 0,
                     static_cast<hipStream_t>(stream), params);
  return static_cast<int>(hipGetLastError());
}

}  // namespace radix_topk_amd
