// Parity oracle for the batched fp16 top-k path.
//
// TEST INFRASTRUCTURE ONLY.  This file is a CPU restatement of the reference's host
// verifier and codec.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
// leg may load it, and only as the checker (or the timed CPU baseline).  The product path
// (batch_topk_amd/) never links, loads or calls it.
//
// What each function restates (reference paths are relative to the reference checkout):
//   oracle_normalize_half_bits   include/type_codec.cuh:13-23
//   oracle_encode_half_asc       include/type_codec.cuh:25-34
//   oracle_encode_half_desc      include/type_codec.cuh:36-38
//   oracle_candidate_better      include/batch_topk_types.cuh:100-113
//   oracle_cpu_reference_topk    include/batch_topk_types.cuh:50-92
//   oracle_simulate_radix_boundary        src/radix_select_state.cuh:9-51
//   oracle_select_high_byte_boundary      src/radix_boundary_select.cuh:9-46
//   oracle_finalize_cutoff_key            src/radix_boundary_select.cuh:48-78
//   oracle_batch_topk_half       the per-segment verifier loop of test/test_batch_topk.cu:566-592
//                                (values re-read raw from the input, as the kernels do in
//                                src/final_topk50.cuh:36 and src/final_block_sort.cuh:66)
//   oracle_make_random_input     test/test_batch_topk.cu:446-454 (std::mt19937 +
//                                std::uniform_real_distribution<float>(-64, 64) + RNE to half)
//
// Pinning (what checks each function against something other than itself) is listed in
// the header comment of oracle/oracle.py and exercised by tests/test_oracle.py.
//
// Extensions beyond the reference (documented decisions, not restatements):
//   * bfloat16 segments (oracle_batch_topk_bf16): the same verifier on the exact
//     bfloat16 -> float widening (the 16 bits become the float's high half), so the
//     reference's comparator applies unchanged; its key (oracle_encode_bf16_desc) is the
//     reference codec's pattern with bfloat16's inf/NaN boundary (0x7F80);
//   * fp32 segments (oracle_batch_topk_f32): the verifier on the floats themselves, the
//     reference comparator's own operand type; values are the raw 32-bit input patterns and
//     pads are index -1 with bits 0xFFFFFFFF;
//   * variable-length segments given by an int64 offset array;
//   * ranks >= min(k, len) of a short segment are padded with index -1 and value bits 0xFFFF.

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>
#include <thread>
#include <vector>

namespace {

// Exact IEEE-754 binary16 -> binary32 widening (what __half2float computes).
float half_bits_to_float(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  uint32_t out;
  if (exp == 0) {
    if (man == 0) {
      out = sign;
    } else {
      // subnormal: value = man * 2^-24; normalise.
      int e = -1;
      uint32_t m = man;
      do {
        ++e;
        m <<= 1;
      } while ((m & 0x400u) == 0);
      out = sign | (static_cast<uint32_t>(127 - 15 - e) << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (exp == 0x1f) {
    out = sign | 0x7f800000u | (man << 13);  // inf / NaN (payload kept)
  } else {
    out = sign | ((exp + 127 - 15) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &out, sizeof(f));
  return f;
}

// Exact bfloat16 -> binary32 widening: bfloat16 is the high half of a binary32.
float bf16_bits_to_float(uint16_t h) {
  const uint32_t out = static_cast<uint32_t>(h) << 16;
  float f;
  std::memcpy(&f, &out, sizeof(f));
  return f;
}

// binary32 -> binary16, round to nearest even (what __float2half computes).
uint16_t float_to_half_rne(float f) {
  uint32_t x;
  std::memcpy(&x, &f, sizeof(x));
  const uint16_t sign = static_cast<uint16_t>((x >> 16) & 0x8000u);
  const uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xff) {
    if (man == 0) return sign | 0x7c00u;
    // NaN: keep the top payload bits, force quiet.
    return static_cast<uint16_t>(sign | 0x7e00u | (man >> 13));
  }
  const int e = static_cast<int>(exp) - 127 + 15;
  if (e >= 0x1f) return sign | 0x7c00u;  // overflow -> inf
  if (e <= 0) {
    // subnormal or zero in half precision
    if (e < -10) return sign;  // rounds to zero (|x| < 2^-25 keeps sign zero)
    man |= 0x800000u;          // implicit bit
    const int shift = 14 - e;  // 1 - e + 13
    const uint32_t q = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    uint32_t r = q;
    if (rem > half || (rem == half && (q & 1u))) ++r;
    return static_cast<uint16_t>(sign | r);
  }
  uint32_t q = man >> 13;
  const uint32_t rem = man & 0x1fffu;
  uint32_t r = (static_cast<uint32_t>(e) << 10) | q;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++r;  // may carry into exponent / inf
  return static_cast<uint16_t>(sign | r);
}

uint16_t normalize_half_bits(uint16_t bits) {
  // include/type_codec.cuh:13-23 -- NaN (any sign/payload) -> 0xffff, +-0 -> 0x0000.
  if ((bits & 0x7c00u) == 0x7c00u && (bits & 0x03ffu) != 0) return 0xffffu;
  if ((bits & 0x7fffu) == 0) return 0x0000u;
  return bits;
}

uint16_t encode_half_asc(uint16_t raw) {
  // include/type_codec.cuh:25-34
  const uint16_t bits = normalize_half_bits(raw);
  return (bits & 0x8000u) ? static_cast<uint16_t>(~bits) : static_cast<uint16_t>(bits ^ 0x8000u);
}

uint16_t encode_half_desc(uint16_t raw) {
  // include/type_codec.cuh:36-38
  return static_cast<uint16_t>(~encode_half_asc(raw));
}

// The codec's pattern (include/type_codec.cuh:13-38) with bfloat16's boundary: NaN (exponent
// all ones, mantissa nonzero; any sign or payload) -> 0xffff, +-0 -> 0x7fff, negative -> bits,
// positive -> bits ^ 0x7fff.
uint16_t encode_bf16_desc(uint16_t raw) {
  if ((raw & 0x7f80u) == 0x7f80u && (raw & 0x007fu) != 0) return 0xffffu;
  if ((raw & 0x7fffu) == 0) return 0x7fffu;
  return (raw & 0x8000u) ? raw : static_cast<uint16_t>(raw ^ 0x7fffu);
}

// include/batch_topk_types.cuh:50-92, operating on the float vector the reference builds.
int cpu_reference_topk(const float* values, int n_values, int seg_len, int k, float* out_values,
                       int* out_indices) {
  if (seg_len <= 0 || k <= 0) return 0;
  const int bounded_seg_len = std::min(seg_len, n_values);
  if (bounded_seg_len <= 0) return 0;
  const int actual_k = std::min(k, bounded_seg_len);
  std::vector<int> order(static_cast<size_t>(bounded_seg_len));
  for (int i = 0; i < bounded_seg_len; ++i) order[static_cast<size_t>(i)] = i;
  std::stable_sort(order.begin(), order.end(), [&](int lhs, int rhs) {
    const float lhs_value = values[lhs];
    const float rhs_value = values[rhs];
    const bool lhs_nan = std::isnan(lhs_value);
    const bool rhs_nan = std::isnan(rhs_value);
    if (lhs_nan != rhs_nan) return rhs_nan;
    if (!lhs_nan && lhs_value != rhs_value) return lhs_value > rhs_value;
    return lhs < rhs;
  });
  for (int i = 0; i < actual_k; ++i) {
    const int index = order[static_cast<size_t>(i)];
    if (out_values) out_values[i] = values[index];
    if (out_indices) out_indices[i] = index;
  }
  return actual_k;
}

// Same ordering as cpu_reference_topk, but with std::partial_sort instead of the full
// std::stable_sort.  The comparator is a strict total order (index breaks every tie), so
// the first actual_k entries are identical; only the running time differs.
int cpu_partial_sort_topk(const float* values, int n_values, int k, int* out_indices,
                          std::vector<int>& order) {
  const int actual_k = std::min(k, n_values);
  if (actual_k <= 0) return 0;
  order.resize(static_cast<size_t>(n_values));
  for (int i = 0; i < n_values; ++i) order[static_cast<size_t>(i)] = i;
  std::partial_sort(order.begin(), order.begin() + actual_k, order.end(), [&](int lhs, int rhs) {
    const float lhs_value = values[lhs];
    const float rhs_value = values[rhs];
    const bool lhs_nan = std::isnan(lhs_value);
    const bool rhs_nan = std::isnan(rhs_value);
    if (lhs_nan != rhs_nan) return rhs_nan;
    if (!lhs_nan && lhs_value != rhs_value) return lhs_value > rhs_value;
    return lhs < rhs;
  });
  for (int i = 0; i < actual_k; ++i) out_indices[i] = order[static_cast<size_t>(i)];
  return actual_k;
}

struct SegmentState {
  // Field order of SegmentSelectState (include/batch_topk_types.cuh:36-45), widened to int.
  int32_t prefix = 0;
  int32_t prefix_mask = 0;
  int32_t cutoff_key = 0xffff;
  int32_t selected_count = 0;
  int32_t live_count = 0;
  int32_t boundary_digit = 0;
  int32_t strictly_better_count = 0;
  int32_t remaining_slots = 0;
};

void store_state(const SegmentState& s, int32_t* out) {
  out[0] = s.prefix;
  out[1] = s.prefix_mask;
  out[2] = s.cutoff_key;
  out[3] = s.selected_count;
  out[4] = s.live_count;
  out[5] = s.boundary_digit;
  out[6] = s.strictly_better_count;
  out[7] = s.remaining_slots;
}

SegmentState load_state(const int32_t* in) {
  SegmentState s;
  s.prefix = in[0];
  s.prefix_mask = in[1];
  s.cutoff_key = in[2];
  s.selected_count = in[3];
  s.live_count = in[4];
  s.boundary_digit = in[5];
  s.strictly_better_count = in[6];
  s.remaining_slots = in[7];
  return s;
}

using ToFloat = float (*)(uint16_t);

void segment_topk_raw(const uint16_t* seg, int64_t len, int k, uint16_t* out_vals,
                      int32_t* out_idx, std::vector<float>& scratch_f, std::vector<int>& scratch_i,
                      ToFloat to_float) {
  // One segment of the verifier loop: 16-bit float -> float (exact), cpu_reference_topk,
  // value re-read raw from the input.  Ranks beyond min(k, len) get the pad (index -1, 0xFFFF).
  int got = 0;
  if (len > 0) {
    scratch_f.resize(static_cast<size_t>(len));
    for (int64_t i = 0; i < len; ++i) scratch_f[static_cast<size_t>(i)] = to_float(seg[i]);
    scratch_i.resize(static_cast<size_t>(std::min<int64_t>(k, len)));
    got = cpu_reference_topk(scratch_f.data(), static_cast<int>(len), static_cast<int>(len), k,
                             nullptr, scratch_i.data());
  }
  for (int r = 0; r < k; ++r) {
    if (r < got) {
      const int idx = scratch_i[static_cast<size_t>(r)];
      out_idx[r] = idx;
      out_vals[r] = seg[idx];
    } else {
      out_idx[r] = -1;
      out_vals[r] = 0xffffu;
    }
  }
}

void segment_bounds(const int64_t* offsets, int64_t seg_len, int s, int64_t* b, int64_t* e) {
  if (offsets) {
    *b = offsets[s];
    *e = offsets[s + 1];
    if (*e < *b) *e = *b;
  } else {
    *b = static_cast<int64_t>(s) * seg_len;
    *e = *b + seg_len;
  }
}

}  // namespace

extern "C" {

uint16_t oracle_normalize_half_bits(uint16_t bits) { return normalize_half_bits(bits); }
uint16_t oracle_encode_half_asc(uint16_t bits) { return encode_half_asc(bits); }
uint16_t oracle_encode_half_desc(uint16_t bits) { return encode_half_desc(bits); }
float oracle_half_to_float(uint16_t bits) { return half_bits_to_float(bits); }
uint16_t oracle_float_to_half(float f) { return float_to_half_rne(f); }
uint16_t oracle_encode_bf16_desc(uint16_t bits) { return encode_bf16_desc(bits); }

void oracle_bf16_to_float_array(const uint16_t* in, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = bf16_bits_to_float(in[i]);
}

void oracle_half_to_float_array(const uint16_t* in, int64_t n, float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = half_bits_to_float(in[i]);
}

void oracle_float_to_half_array(const float* in, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = float_to_half_rne(in[i]);
}

// include/batch_topk_types.cuh:100-113 on (raw half bits, index) pairs.
int oracle_candidate_better(uint16_t lhs_bits, int lhs_index, uint16_t rhs_bits, int rhs_index) {
  const float lhs_value = half_bits_to_float(lhs_bits);
  const float rhs_value = half_bits_to_float(rhs_bits);
  const bool lhs_nan = lhs_value != lhs_value;
  const bool rhs_nan = rhs_value != rhs_value;
  if (lhs_nan != rhs_nan) return rhs_nan ? 1 : 0;
  if (!lhs_nan && lhs_value != rhs_value) return lhs_value > rhs_value ? 1 : 0;
  return lhs_index < rhs_index ? 1 : 0;
}

int oracle_cpu_reference_topk(const float* values, int n_values, int seg_len, int k,
                              float* out_values, int* out_indices) {
  return cpu_reference_topk(values, n_values, seg_len, k, out_values, out_indices);
}

// src/radix_select_state.cuh:9-51 (the input floats go through __float2half first, as there).
void oracle_simulate_radix_boundary(const float* values, int n_values, int seg_len, int k,
                                    int32_t* state_out) {
  SegmentState state;
  if (seg_len <= 0 || k <= 0) {
    store_state(state, state_out);
    return;
  }
  const int bounded_seg_len = std::min(seg_len, n_values);
  if (bounded_seg_len <= 0) {
    store_state(state, state_out);
    return;
  }
  std::vector<int> counts(256, 0);
  for (int i = 0; i < bounded_seg_len; ++i) {
    const uint16_t encoded = encode_half_desc(float_to_half_rne(values[i]));
    ++counts[(encoded >> 8) & 0xffu];
  }
  const int actual_k = std::min(k, bounded_seg_len);
  int selected_count = 0;
  int boundary_digit = 0;
  int live_count = counts[0];
  for (int bucket = 0; bucket < 256; ++bucket) {
    const int bucket_count = counts[static_cast<size_t>(bucket)];
    if (selected_count + bucket_count < actual_k) {
      selected_count += bucket_count;
      continue;
    }
    boundary_digit = bucket;
    live_count = bucket_count;
    break;
  }
  state.prefix = (boundary_digit << 8) & 0xffff;
  state.prefix_mask = 0xff00;
  state.selected_count = selected_count;
  state.live_count = live_count;
  state.boundary_digit = boundary_digit;
  store_state(state, state_out);
}

// src/radix_boundary_select.cuh:9-46 for one segment's 256-bin high-byte histogram.
void oracle_select_high_byte_boundary(const uint32_t* histogram, int k, int32_t* state_out) {
  SegmentState state;
  int selected = 0;
  for (int bucket = 0; bucket < 256; ++bucket) {
    const int count = static_cast<int>(histogram[bucket]);
    if (selected + count < k) {
      selected += count;
      continue;
    }
    state.boundary_digit = bucket;
    state.prefix = (bucket << 8) & 0xffff;
    state.prefix_mask = 0xff00;
    state.selected_count = selected;
    state.live_count = count;
    store_state(state, state_out);
    return;
  }
  state.prefix = 0xffff;
  state.prefix_mask = 0xffff;
  state.cutoff_key = 0xffff;
  state.selected_count = selected;
  state.live_count = 0;
  state.boundary_digit = 255;
  state.strictly_better_count = selected;
  state.remaining_slots = (k > selected) ? (k - selected) : 0;
  store_state(state, state_out);
}

// src/radix_boundary_select.cuh:48-78: continue the cumulative count over the low byte.
void oracle_finalize_cutoff_key(const uint32_t* histogram_lo, int k, int32_t* state_io) {
  SegmentState state = load_state(state_io);
  int selected = state.selected_count;
  for (int bucket = 0; bucket < 256; ++bucket) {
    const int count = static_cast<int>(histogram_lo[bucket]);
    if (selected + count < k) {
      selected += count;
      continue;
    }
    state.cutoff_key = ((state.boundary_digit << 8) | bucket) & 0xffff;
    state.strictly_better_count = selected;
    state.remaining_slots = k - selected;
    store_state(state, state_io);
    return;
  }
  state.cutoff_key = 0xffff;
  state.strictly_better_count = selected;
  state.remaining_slots = (k > selected) ? (k - selected) : 0;
  store_state(state, state_io);
}

// Histogram of (key >> shift) & 0xff over keys whose (key & mask) == prefix
// (src/radix_histogram.cuh:158-186, the generic pass the reference tests use).
void oracle_histogram_pass(const uint16_t* input, int n, int shift, uint16_t prefix, uint16_t mask,
                           uint32_t* histogram) {
  for (int b = 0; b < 256; ++b) histogram[b] = 0;
  for (int i = 0; i < n; ++i) {
    const uint16_t key = encode_half_desc(input[i]);
    if ((key & mask) == prefix) ++histogram[(key >> shift) & 0xffu];
  }
}

// Runs run(s_begin, s_end) over the segments, serially when threads <= 1 (exactly like the
// reference harness loop), else split over `threads` host threads.
extern "C++" template <class Run>
void over_segments(int seg_num, int threads, Run run) {
  if (threads <= 1 || seg_num == 1) {
    run(0, seg_num);
    return;
  }
  const int nt = std::min(threads, seg_num);
  std::vector<std::thread> pool;
  for (int t = 0; t < nt; ++t) {
    const int b = static_cast<int>(static_cast<int64_t>(seg_num) * t / nt);
    const int e = static_cast<int>(static_cast<int64_t>(seg_num) * (t + 1) / nt);
    pool.emplace_back(run, b, e);
  }
  for (auto& th : pool) th.join();
}

// Batched verifier: for each segment, the reference's cpu_reference_topk on the exact
// float widening of the fp16 input; values are written as the raw input bits at the
// selected index.  offsets == nullptr selects fixed-length segments of seg_len.
static int batch_topk_16(const uint16_t* input, const int64_t* offsets, int seg_num,
                         int64_t seg_len, int k, uint16_t* out_vals, int32_t* out_idx,
                         int threads, ToFloat to_float) {
  if (seg_num <= 0 || k <= 0) return 1;
  over_segments(seg_num, threads, [&](int s_begin, int s_end) {
    std::vector<float> f;
    std::vector<int> idx;
    for (int s = s_begin; s < s_end; ++s) {
      int64_t b, e;
      segment_bounds(offsets, seg_len, s, &b, &e);
      segment_topk_raw(input + b, e - b, k, out_vals + static_cast<int64_t>(s) * k,
                       out_idx + static_cast<int64_t>(s) * k, f, idx, to_float);
    }
  });
  return 0;
}

// fp32 segments: cpu_reference_topk on the floats themselves (its comparator's own operand
// type); values are the raw 32-bit input patterns at the selected index, pads index -1 with
// bits 0xFFFFFFFF.
int oracle_batch_topk_f32(const uint32_t* input, const int64_t* offsets, int seg_num,
                          int64_t seg_len, int k, uint32_t* out_vals, int32_t* out_idx,
                          int threads) {
  if (seg_num <= 0 || k <= 0) return 1;
  over_segments(seg_num, threads, [&](int s_begin, int s_end) {
    std::vector<float> f;
    std::vector<int> idx;
    for (int s = s_begin; s < s_end; ++s) {
      int64_t b, e;
      segment_bounds(offsets, seg_len, s, &b, &e);
      const int64_t len = e - b;
      uint32_t* ov = out_vals + static_cast<int64_t>(s) * k;
      int32_t* oi = out_idx + static_cast<int64_t>(s) * k;
      int got = 0;
      if (len > 0) {
        f.resize(static_cast<size_t>(len));
        std::memcpy(f.data(), input + b, static_cast<size_t>(len) * 4);
        idx.resize(static_cast<size_t>(std::min<int64_t>(k, len)));
        got = cpu_reference_topk(f.data(), static_cast<int>(len), static_cast<int>(len), k, nullptr,
                                 idx.data());
      }
      for (int r = 0; r < k; ++r) {
        oi[r] = r < got ? idx[static_cast<size_t>(r)] : -1;
        ov[r] = r < got ? input[b + idx[static_cast<size_t>(r)]] : 0xffffffffu;
      }
    }
  });
  return 0;
}

int oracle_batch_topk_half(const uint16_t* input, const int64_t* offsets, int seg_num,
                           int64_t seg_len, int k, uint16_t* out_vals, int32_t* out_idx,
                           int threads) {
  return batch_topk_16(input, offsets, seg_num, seg_len, k, out_vals, out_idx, threads,
                       half_bits_to_float);
}

// The same verifier on bfloat16 segments (exact widening to float, the same comparator).
int oracle_batch_topk_bf16(const uint16_t* input, const int64_t* offsets, int seg_num,
                           int64_t seg_len, int k, uint16_t* out_vals, int32_t* out_idx,
                           int threads) {
  return batch_topk_16(input, offsets, seg_num, seg_len, k, out_vals, out_idx, threads,
                       bf16_bits_to_float);
}

// CPU baseline timing: runs the verifier over segments [0, seg_count) `reps` times and
// returns the median wall time in seconds.  variant 0 = stable_sort (the reference's code),
// variant 1 = partial_sort (identical output).
double oracle_time_batch_topk_half(const uint16_t* input, const int64_t* offsets, int seg_count,
                                   int64_t seg_len, int k, int threads, int variant, int reps,
                                   int32_t* out_idx) {
  std::vector<double> times;
  std::vector<uint16_t> vals(static_cast<size_t>(seg_count) * static_cast<size_t>(k));
  for (int r = 0; r < std::max(1, reps); ++r) {
    const auto t0 = std::chrono::steady_clock::now();
    if (variant == 0) {
      oracle_batch_topk_half(input, offsets, seg_count, seg_len, k, vals.data(), out_idx, threads);
    } else {
      auto run = [&](int s_begin, int s_end) {
        std::vector<float> f;
        std::vector<int> order;
        for (int s = s_begin; s < s_end; ++s) {
          int64_t b, e;
          segment_bounds(offsets, seg_len, s, &b, &e);
          const int64_t len = e - b;
          f.resize(static_cast<size_t>(len));
          for (int64_t i = 0; i < len; ++i) f[static_cast<size_t>(i)] = half_bits_to_float(input[b + i]);
          int32_t* o = out_idx + static_cast<int64_t>(s) * k;
          const int got = cpu_partial_sort_topk(f.data(), static_cast<int>(len), k, o, order);
          for (int q = got; q < k; ++q) o[q] = -1;
        }
      };
      if (threads <= 1 || seg_count == 1) {
        run(0, seg_count);
      } else {
        const int nt = std::min(threads, seg_count);
        std::vector<std::thread> pool;
        for (int t = 0; t < nt; ++t) {
          const int b = static_cast<int>(static_cast<int64_t>(seg_count) * t / nt);
          const int e = static_cast<int>(static_cast<int64_t>(seg_count) * (t + 1) / nt);
          pool.emplace_back(run, b, e);
        }
        for (auto& th : pool) th.join();
      }
    }
    const auto t1 = std::chrono::steady_clock::now();
    times.push_back(std::chrono::duration<double>(t1 - t0).count());
  }
  std::sort(times.begin(), times.end());
  return times[times.size() / 2];
}

// test/test_batch_topk.cu:446-454: std::mt19937(seed) + uniform_real_distribution<float>(-64,64),
// each draw rounded through half.  Writes the rounded floats and the raw half bits.
void oracle_make_random_input(int seg_num, int seg_len, uint32_t seed, float* out_values,
                              uint16_t* out_bits) {
  std::mt19937 rng(seed);
  std::uniform_real_distribution<float> dist(-64.0f, 64.0f);
  const int64_t n = static_cast<int64_t>(seg_num) * seg_len;
  for (int64_t i = 0; i < n; ++i) {
    const uint16_t h = float_to_half_rne(dist(rng));
    if (out_bits) out_bits[i] = h;
    if (out_values) out_values[i] = half_bits_to_float(h);
  }
}

}  // extern "C"
