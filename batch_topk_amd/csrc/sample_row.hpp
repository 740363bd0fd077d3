// One top-k sampling draw per row, shared by the fused path (the top-k kernel's last step,
// ranked entries in LDS) and the stand-alone sampling kernel (entries in global memory).
//
// For a row whose top-k values in rank order are v_0 >= v_1 >= ... (m valid ranks):
//   w_0 = 1;  for r >= 1: w_r = 1 if v_r == v_0, else exp((v_r - v_0) * inv_t), and 0 when
//   that is NaN (a NaN logit); a finite v_r below v_0 = +inf gets exp(-inf) = 0;
//   S = w_0 + ... + w_{m-1} (fp32);  the sample is the index at the first rank r whose
//   running sum w_0 + ... + w_r exceeds u * S (the last rank if rounding leaves none), and
//   probs[r] = w_r / S (0 for r >= m).  An empty row (m = 0) samples index -1.
// inv_t is 1 / temperature rounded to fp32 on the host.  Equal logits get equal weight, so
// -inf logits weigh 0 unless every rank is -inf.
//
// Each lane of the calling wave owns a contiguous run of ceil(k / 64) ranks: it computes their
// weights and its run's sum, a wave prefix sum gives every run its start, and the first lane
// whose run crosses u * S picks the rank inside its run.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "topk_common.hpp"

namespace radix_topk_amd {

// Exact widening of a 16-bit float (fp16, or bfloat16 when bf16) to float.
__device__ __forceinline__ float bits16_to_float(uint32_t b, bool bf16) {
  if (bf16) return __uint_as_float(b << 16);
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(b)));
}

namespace sample_detail {

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, ROW_MASK, 0xf, false);
}

// Inclusive prefix sums across a wave64: DPP row shifts, then the row broadcasts carry row
// totals upward.
__device__ __forceinline__ float wave_scan(float x) {
  x += __int_as_float(dpp_i<0x111, 0xf>(__float_as_int(x)));
  x += __int_as_float(dpp_i<0x112, 0xf>(__float_as_int(x)));
  x += __int_as_float(dpp_i<0x114, 0xf>(__float_as_int(x)));
  x += __int_as_float(dpp_i<0x118, 0xf>(__float_as_int(x)));
  x += __int_as_float(dpp_i<0x142, 0xa>(__float_as_int(x)));
  x += __int_as_float(dpp_i<0x143, 0xc>(__float_as_int(x)));
  return x;
}

}  // namespace sample_detail

constexpr int kSampleMaxRun = (kMaxTopK + 63) / 64;  // ranks per lane at the largest k

// Called by one whole wave.  get(r) returns the rank-r entry as {value (float), index} for
// r < m.  Writes *sample_out (lane 0) and, when probs_row is not null, probs_row[0..k).
template <class Get>
__device__ void sample_ranked_row(Get get, int m, int k, float inv_t, float u, int32_t* sample_out,
                                  float* probs_row) {
  const int lane = threadIdx.x & 63;
  if (m <= 0) {
    if (lane == 0) *sample_out = -1;
    if (probs_row) {
      for (int r = lane; r < k; r += 64) probs_row[r] = 0.0f;
    }
    return;
  }
  const int run = (k + 63) / 64;
  const int r0 = lane * run;
  const float v0 = get(0).value;
  float w[kSampleMaxRun];
  float lane_sum = 0.0f;
#pragma unroll
  for (int t = 0; t < kSampleMaxRun; ++t) {
    w[t] = 0.0f;
    const int r = r0 + t;
    if (t < run && r < m) {
      const float v = get(r).value;
      float x = (r == 0 || v == v0) ? 1.0f : expf((v - v0) * inv_t);
      if (x != x) x = 0.0f;
      w[t] = x;
      lane_sum += x;
    }
  }
  const float incl = sample_detail::wave_scan(lane_sum);
  const float total = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(incl), 63));
  const float target = u * total;
  float acc = incl - lane_sum;
  int hit = -1;
#pragma unroll
  for (int t = 0; t < kSampleMaxRun; ++t) {
    const int r = r0 + t;
    if (t < run && r < m) {
      acc += w[t];
      if (hit < 0 && acc > target) hit = r;
    }
  }
  const unsigned long long lanes = __builtin_amdgcn_ballot_w64(hit >= 0);
  const int pick = lanes ? __builtin_amdgcn_readlane(hit, static_cast<int>(__builtin_ctzll(lanes))) : m - 1;
  if (lane == 0) *sample_out = get(pick).index;
  if (probs_row) {
    const float inv_total = 1.0f / total;
#pragma unroll
    for (int t = 0; t < kSampleMaxRun; ++t) {
      const int r = r0 + t;
      if (t < run && r < k) probs_row[r] = w[t] * inv_total;
    }
  }
}

struct RankedEntry {
  float value;
  int32_t index;
};

}  // namespace radix_topk_amd
