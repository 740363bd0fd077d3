// Host side of the batched fp16 top-k engine: argument validation, launch planning,
// workspace carve and the C ABI declared in include/batch_topk.h.
//
// Validation runs before any HIP call, so every rejected argument returns
// hipErrorInvalidValue (1) even on a machine without a GPU (reference behaviour:
// src/batch_topk.cu:13-33,51-60).  The plan depends only on (seg_num, segment length, k),
// so the workspace size is pure host arithmetic (reference src/batch_topk.cu:35-40).

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <random>

#include "../../include/batch_topk.h"
#include "topk_common.hpp"

namespace radix_topk_amd {
namespace {

constexpr int kMaxK = RADIX_TOPK_MAX_K;
constexpr size_t kAlign = 256;
// CU count the plan assumes (MI355X).  The plan depends on the shape only; the device's own
// CU count is checked at launch where it matters (the cooperative path).
constexpr int kPlanCUs = 256;
constexpr int kInvalid = static_cast<int>(hipErrorInvalidValue);

int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Launch plan for segments of at most `max_len` elements (plus up to ev - 1 elements of
// misalignment of the 16-byte load grid), `seg_num` segments and `k` outputs each, for
// elements of which one 16-byte vector holds `ev` (8 for 16-bit formats, 4 for fp32).
// `shared_alignment`: fixed-length rows that all start at the input pointer's alignment (one
// row, or a length that is a whole number of vectors), so that the launch knows the exact
// aligned span of every row.
//
// The workgroup shape has at least 4k threads so each wave's share of k stays well below its
// 64 lanes; the rest of the choice depends on how many segments share a CU (below).  Longer segments are split into
// kMaxChunk chunks whose candidate lists are merged by the last workgroup to finish, while
// the W lists fit one workgroup's LDS merge area.  Beyond that (long segments with large k)
// the segment's W workgroups run cooperatively: all co-resident, they build one
// whole-segment threshold from global histograms and a single candidate list.
Plan make_plan(int seg_num, int64_t max_len, int k, int ev = 8, bool shared_alignment = false) {
  Plan plan{};
  plan.ok = false;
  if (seg_num <= 0 || k <= 0 || k > kMaxK || max_len < 0) return plan;
  const int block_min = k <= 64 ? 256 : (k <= 128 ? 512 : 1024);
  const int64_t span = max_len + ev - 1;  // worst-case aligned span of one segment
  int block = 1024, vpt = 16;
  bool found = false;
  if (seg_num >= 2 * kPlanCUs) {
    // More segments than two per CU: the fewest threads (at least 512; 256 for rows that 256
    // threads x 4 vectors cover, or x 8 vectors from three segments per CU on) whose chunk
    // covers max_len, so that several workgroups share a CU and one's loads overlap another's
    // selection.  A segment whose misaligned span reaches past the chunk takes a second (tail)
    // workgroup.  (With fewer segments, 8-vector rows on 256 threads leave too few waves per
    // CU: 512 x 12,000 ran 7.14 us on 512 threads and 7.62 on 256, while 800 x 12,000 ran 10.14
    // and 9.08.  Longer rows on 256 threads take 16 vectors per thread, whose per-wave chains
    // cost more than the extra workgroups gain: 1,024 x 30,000 ran 14.39 us on 512 threads
    // and 14.92 on 256.)
    const bool many_short = max_len <= 256 * 4 * ev || (max_len <= 256 * 8 * ev && seg_num >= 3 * kPlanCUs);
    const int many_min = many_short ? 256 : 512;
    for (int cb = block_min > many_min ? block_min : many_min; cb <= 1024 && !found; cb *= 2) {
      for (int cv : {2, 4, 8, 16}) {
        if (!found && static_cast<int64_t>(cb) * cv * ev >= max_len) {
          block = cb;
          vpt = cv;
          found = true;
        }
      }
    }
  } else {
    // Up to two segments per CU: one workgroup per segment with the fewest vectors per
    // thread (then the fewest threads) that covers the whole aligned span.
    for (int cv : {2, 4, 8, 16}) {
      for (int cb = block_min; cb <= 1024 && !found; cb *= 2) {
        if (static_cast<int64_t>(cb) * cv * ev >= span) {
          block = cb;
          vpt = cv;
          found = true;
        }
      }
      if (found) break;
    }
  }
  int chunk = block * vpt * ev;
  int64_t W = span <= chunk ? 1 : (span + chunk - 1) / chunk;
  const int kpad = next_pow2(k < 64 ? 64 : k);
  int cap_list = W > 1 ? next_pow2(2 * k > 128 ? 2 * k : 128) : 0;
  bool cooperative = false;
  int group = 0;
  if (W > 1 && W * static_cast<int64_t>(cap_list) > kCandArea) {
    // Too many lists to merge in LDS: one whole-segment threshold, over chunks of 1024 threads x
    // 16 vectors (a segment that then fits one chunk is a plain single-chunk row).
    block = 1024;
    vpt = 16;
    chunk = block * vpt * ev;
    W = span <= chunk ? 1 : (span + chunk - 1) / chunk;
    cap_list = 0;
    if (W > 1) {
      // The cooperative path (one workgroup per chunk, all co-resident) when the grid fits the
      // CUs.  The workspace covers the worst-case misalignment (W chunks).  Rows of a shared
      // alignment launch with their exact chunk count, ceil(max_len / chunk) when 16-byte
      // aligned (a misaligned pointer that needs more co-resident workgroups is refused at
      // launch).
      const int64_t w_launch = shared_alignment ? (max_len + chunk - 1) / chunk : W;
      if (static_cast<int64_t>(seg_num) * w_launch <= kMaxCoopGroups) {
        cooperative = true;
        // Half-length chunks (8 vectors per thread) when that grid fits too: twice as many CUs
        // pull the segment in (a CU keeps about 64 KB of loads in flight, so 256 KB per CU
        // arrive in four rounds and 128 KB in two).
        const int chunk8 = 1024 * 8 * ev;
        const int64_t W8 = (span + chunk8 - 1) / chunk8;
        const int64_t w_launch8 = shared_alignment ? (max_len + chunk8 - 1) / chunk8 : W8;
        if (static_cast<int64_t>(seg_num) * w_launch8 <= kMaxCoopGroups) {
          vpt = 8;
          chunk = chunk8;
          W = W8;
        }
      } else {
        // The long-segment path: `group` workgroups per segment, each taking every group-th
        // chunk of it, as many per segment as the CUs hold at once for few segments, one per
        // segment (no waiting across workgroups) otherwise.
        group = seg_num <= kMaxCoopGroups ? static_cast<int>(std::min<int64_t>(W, kMaxCoopGroups / seg_num)) : 1;
      }
    }
  }
  if (static_cast<int64_t>(seg_num) * W > 0x7fffffff) return plan;

  plan.shape = KernelShape{block, vpt};
  plan.chunk = chunk;
  plan.W = static_cast<int>(W);
  plan.cap_chunk = kCandArea;
  plan.cap_list = cap_list;
  plan.cand_area = kCandArea;
  plan.kpad = kpad;
  const int rank_cap = kpad > 512 ? kpad : 512;
  plan.lds_bytes = 256 * 4 + 256 * 4 + 32 * 4 + 16 * 4 + static_cast<size_t>(kCandArea) * 8 +
                   static_cast<size_t>(kpad) * 8 + static_cast<size_t>(rank_cap) * 4 +
                   static_cast<size_t>(block / 64) * kStageWords * 4;
  plan.cooperative = cooperative;
  plan.group = group;
  size_t ws = kAlign;                                        // alignment slack of the carve
  ws += align_up(static_cast<size_t>(seg_num) * 8, kAlign);  // arrival tickets
  ws += align_up(static_cast<size_t>(seg_num) * 4, kAlign);  // per-segment status words
  if (cooperative) {
    ws += static_cast<size_t>(seg_num) * group_layout(static_cast<int>(W)).bytes;  // group blocks
  } else if (group > 1) {
    // (one workgroup per segment keeps its histograms and list in LDS: no block)
    ws += static_cast<size_t>(seg_num) * group_layout(group).bytes;
  } else if (W > 1) {
    ws += align_up(static_cast<size_t>(seg_num) * W * 4, kAlign);               // list counts
    ws += static_cast<size_t>(seg_num) * W * static_cast<size_t>(cap_list) * 8;  // lists
  }
  plan.ws_bytes = ws;
  plan.ok = true;
  return plan;
}

// Process-wide source of 48-bit call tokens for the arrival counters.  Tokens never repeat
// within a process, start at a random point, and skip values whose six bytes are all equal
// (the shape of a memset-poisoned workspace word).
uint64_t next_epoch() {
  static std::atomic<uint64_t> counter{[] {
    std::random_device rd;
    const uint64_t t = static_cast<uint64_t>(
        std::chrono::steady_clock::now().time_since_epoch().count());
    return ((static_cast<uint64_t>(rd()) << 32) ^ static_cast<uint64_t>(rd()) ^ (t * 0x9E3779B97F4A7C15ull));
  }()};
  for (;;) {
    const uint64_t e = counter.fetch_add(1, std::memory_order_relaxed) & 0xFFFFFFFFFFFFull;
    const uint64_t b = e & 0xff;
    if (e == 0 || e == b * 0x010101010101ull) continue;
    return e;
  }
}

// Test hook of the bounded cross-workgroup waits: spin limit << 32 | kForce* bits, or 0 for
// ordinary calls (radix_topk_debug_wait_hook).
std::atomic<uint64_t> g_wait_hook{0};

// Top-k sampling request riding on a top-k call (sample_topk).
struct SampleSpec {
  const float* uniforms;
  int32_t* samples;
  float* probs;
  float inv_temperature;
};

int run(const Plan& plan, uint32_t inf_bits, const void* d_input, const int32_t* d_offsets,
        int seg_num, int64_t seg_len, int64_t max_len, int k, void* d_values, int32_t* d_indices,
        void* d_workspace, size_t workspace_bytes, void* stream, const SampleSpec* sample = nullptr,
        bool unsorted = false) {
  if (!plan.ok || workspace_bytes < plan.ws_bytes) return kInvalid;
  const uintptr_t in_addr = reinterpret_cast<uintptr_t>(d_input);
  const uintptr_t eb = inf_bits == kInfBitsF32 ? 4u : 2u;  // element bytes
  if ((in_addr % eb) || (reinterpret_cast<uintptr_t>(d_values) % eb) ||
      (reinterpret_cast<uintptr_t>(d_indices) & 3u) || (reinterpret_cast<uintptr_t>(d_offsets) & 3u)) {
    return kInvalid;
  }
  TopkParams p{};
  p.base = reinterpret_cast<const uint16_t*>(in_addr & ~static_cast<uintptr_t>(15));
  p.elem0 = static_cast<int64_t>((in_addr & 15u) / eb);
  p.elem_bytes = static_cast<int32_t>(eb);
  p.offsets = d_offsets;
  p.seg_len = seg_len;
  p.max_len = max_len;
  p.seg_num = seg_num;
  p.k = k;
  p.chunks_per_seg = plan.W;
  if (plan.cooperative && !d_offsets) {
    // Fixed-length rows that all share the input pointer's alignment (one row, or a length
    // that is a whole number of 16-byte vectors): the exact aligned span decides the chunk
    // count, so an aligned row does not pay a workgroup for the worst-case misalignment.
    const int64_t ev = 16 / static_cast<int64_t>(eb);
    if (seg_num == 1 || seg_len % ev == 0) {
      const int64_t span = p.elem0 + seg_len;
      p.chunks_per_seg = static_cast<int32_t>((span + plan.chunk - 1) / plan.chunk);
    }
  }
  p.cap_chunk = plan.cap_chunk;
  p.cap_list = plan.cap_list;
  p.cand_area = plan.cand_area;
  p.kpad = plan.kpad;
  p.out_vals = d_values;  // nullptr: indices only
  p.unsorted = unsorted ? 1 : 0;
  p.out_idx = d_indices;
  const uintptr_t ws = align_up(reinterpret_cast<uintptr_t>(d_workspace), kAlign);
  size_t off = 0;
  p.tickets = reinterpret_cast<unsigned long long*>(ws + off);
  off += align_up(static_cast<size_t>(seg_num) * 8, kAlign);
  p.status = reinterpret_cast<uint32_t*>(ws + off);
  off += align_up(static_cast<size_t>(seg_num) * 4, kAlign);
  p.cooperative = plan.cooperative ? 1 : 0;
  p.group = plan.group;
  if (plan.cooperative || plan.group > 0) {
    p.groups = reinterpret_cast<unsigned char*>(ws + off);
  } else if (plan.W > 1) {
    p.list_counts = reinterpret_cast<int32_t*>(ws + off);
    off += align_up(static_cast<size_t>(seg_num) * plan.W * 4, kAlign);
    p.lists = reinterpret_cast<unsigned long long*>(ws + off);
  }
  p.epoch = next_epoch();
  p.inf_bits = inf_bits;
  const uint64_t hook = g_wait_hook.load(std::memory_order_relaxed);
  p.spin_limit = hook ? static_cast<uint32_t>(hook >> 32) : kDefaultSpinLimit;
  p.force_timeout = static_cast<uint32_t>(hook);
  // Sampling is fused into the kernel's last step, except on the whole-segment plans
  // (cooperative or long-segment: the ranking is spread over the segment's workgroups): there a
  // one-wave-per-row kernel follows.
  const bool whole_segment = plan.cooperative || plan.group > 0;
  if (sample && !whole_segment) {
    p.uniforms = sample->uniforms;
    p.samples = sample->samples;
    p.probs = sample->probs;
    p.inv_temperature = sample->inv_temperature;
  }
  const int rc = launch_segmented_topk(plan, p, stream);
  if (rc != 0 || !sample || !whole_segment) return rc;
  SampleParams sp{};
  sp.topk_vals = static_cast<const uint16_t*>(d_values);
  sp.topk_idx = d_indices;
  sp.uniforms = sample->uniforms;
  sp.samples = sample->samples;
  sp.probs = sample->probs;
  sp.inv_temperature = sample->inv_temperature;
  sp.seg_num = seg_num;
  sp.k = k;
  sp.bf16 = inf_bits == kInfBitsBF16 ? 1 : 0;
  return launch_topk_sample(sp, stream);
}

// Elements per 16-byte vector of the format whose +inf pattern is `inf_bits`.
int ev_of(uint32_t inf_bits) { return inf_bits == kInfBitsF32 ? 4 : 8; }

// Fixed-length rows that all start at the input pointer's alignment.
bool shared_alignment(int seg_num, int64_t seg_len, uint32_t inf_bits) {
  return seg_num == 1 || seg_len % ev_of(inf_bits) == 0;
}

size_t fixed_workspace_size(int seg_num, int seg_len, int k, uint32_t inf_bits = kInfBitsF16) {
  if (seg_num <= 0 || seg_len <= 0 || k <= 0 || k > RADIX_TOPK_MAX_K || k > seg_len) return 0;
  const Plan plan =
      make_plan(seg_num, seg_len, k, ev_of(inf_bits), shared_alignment(seg_num, seg_len, inf_bits));
  return plan.ok ? plan.ws_bytes : 0;
}

int fixed_topk(uint32_t inf_bits, const void* d_input, int seg_num, int seg_len, int k,
               void* d_output_values, int32_t* d_output_indices, void* d_workspace,
               size_t workspace_bytes, void* stream) {
  if (seg_num <= 0 || seg_len <= 0 || k <= 0 || k > RADIX_TOPK_MAX_K || k > seg_len) return kInvalid;
  if (!d_input || !d_output_values || !d_output_indices || !d_workspace) return kInvalid;
  const Plan plan =
      make_plan(seg_num, seg_len, k, ev_of(inf_bits), shared_alignment(seg_num, seg_len, inf_bits));
  return run(plan, inf_bits, d_input, nullptr, seg_num, seg_len, seg_len, k, d_output_values,
             d_output_indices, d_workspace, workspace_bytes, stream);
}

size_t segmented_workspace_size(int seg_num, int max_seg_len, int k, uint32_t inf_bits = kInfBitsF16) {
  if (seg_num <= 0 || max_seg_len < 0 || k <= 0 || k > RADIX_TOPK_MAX_K) return 0;
  const Plan plan = make_plan(seg_num, max_seg_len, k, ev_of(inf_bits));
  return plan.ok ? plan.ws_bytes : 0;
}

int segmented_topk(uint32_t inf_bits, const void* d_input, const int32_t* d_offsets, int seg_num,
                   int max_seg_len, int k, void* d_output_values, int32_t* d_output_indices,
                   void* d_workspace, size_t workspace_bytes, void* stream) {
  if (seg_num <= 0 || max_seg_len < 0 || k <= 0 || k > RADIX_TOPK_MAX_K) return kInvalid;
  if (!d_input || !d_offsets || !d_output_values || !d_output_indices || !d_workspace) return kInvalid;
  const Plan plan = make_plan(seg_num, max_seg_len, k, ev_of(inf_bits));
  return run(plan, inf_bits, d_input, d_offsets, seg_num, 0, max_seg_len, k, d_output_values,
             d_output_indices, d_workspace, workspace_bytes, stream);
}

// Extended entry point: element format, fixed-length or segmented input, output flags.
bool known_format(int format) {
  return format == RADIX_TOPK_FORMAT_F16 || format == RADIX_TOPK_FORMAT_BF16 ||
         format == RADIX_TOPK_FORMAT_F32;
}

uint32_t inf_of(int format) {
  return format == RADIX_TOPK_FORMAT_F32 ? kInfBitsF32
                                         : (format == RADIX_TOPK_FORMAT_BF16 ? kInfBitsBF16 : kInfBitsF16);
}

size_t ex_workspace_size(int format, int segmented, int seg_num, int seg_len, int k) {
  if (!known_format(format)) return 0;
  return segmented ? segmented_workspace_size(seg_num, seg_len, k, inf_of(format))
                   : fixed_workspace_size(seg_num, seg_len, k, inf_of(format));
}

int topk_ex(const void* d_input, int format, const int32_t* d_offsets, int seg_num, int seg_len, int k,
            int flags, void* d_output_values, int32_t* d_output_indices, void* d_workspace,
            size_t workspace_bytes, void* stream) {
  if (!known_format(format)) return kInvalid;
  if (flags & ~(RADIX_TOPK_UNSORTED | RADIX_TOPK_INDICES_ONLY)) return kInvalid;
  const bool indices_only = (flags & RADIX_TOPK_INDICES_ONLY) != 0;
  if (seg_num <= 0 || k <= 0 || k > RADIX_TOPK_MAX_K) return kInvalid;
  if (d_offsets ? seg_len < 0 : (seg_len <= 0 || k > seg_len)) return kInvalid;
  if (!d_input || !d_output_indices || !d_workspace || (!indices_only && !d_output_values)) return kInvalid;
  const uint32_t inf = inf_of(format);
  const Plan plan =
      make_plan(seg_num, seg_len, k, ev_of(inf), !d_offsets && shared_alignment(seg_num, seg_len, inf));
  void* vals = indices_only ? nullptr : d_output_values;
  return run(plan, inf, d_input, d_offsets, seg_num, d_offsets ? 0 : seg_len,
             seg_len, k, vals, d_output_indices, d_workspace, workspace_bytes, stream, nullptr,
             (flags & RADIX_TOPK_UNSORTED) != 0);
}

// Top-k of every row, then one draw per row from the softmax of its top-k.
int sample_topk(bool bf16, const uint16_t* d_logits, int seg_num, int seg_len, int k,
                float temperature, const float* d_uniforms, uint16_t* d_topk_values,
                int32_t* d_topk_indices, float* d_probs, int32_t* d_samples, void* d_workspace,
                size_t workspace_bytes, void* stream) {
  if (seg_num <= 0 || seg_len <= 0 || k <= 0 || k > RADIX_TOPK_MAX_K || k > seg_len) return kInvalid;
  if (!d_logits || !d_topk_values || !d_topk_indices || !d_workspace) return kInvalid;
  if (!(temperature > 0.0f) || !std::isfinite(temperature)) return kInvalid;
  if (!d_uniforms || !d_samples) return kInvalid;
  const float inv_t = 1.0f / temperature;
  if (!std::isfinite(inv_t)) return kInvalid;
  const Plan plan = make_plan(seg_num, seg_len, k, 8, shared_alignment(seg_num, seg_len, kInfBitsF16));
  const SampleSpec spec{d_uniforms, d_samples, d_probs, inv_t};
  return run(plan, bf16 ? kInfBitsBF16 : kInfBitsF16, d_logits, nullptr, seg_num, seg_len, seg_len, k,
             d_topk_values, d_topk_indices, d_workspace, workspace_bytes, stream, &spec);
}

// Copies the per-segment status words of the last call made with the workspace (see
// radix_topk_workspace_status in batch_topk.h).
int workspace_status(const void* d_workspace, size_t workspace_bytes, int seg_num, uint32_t* h_status,
                     void* stream) {
  if (!d_workspace || !h_status || seg_num <= 0) return kInvalid;
  const uintptr_t ws = align_up(reinterpret_cast<uintptr_t>(d_workspace), kAlign);
  const size_t off = align_up(static_cast<size_t>(seg_num) * 8, kAlign);
  const size_t need = (ws - reinterpret_cast<uintptr_t>(d_workspace)) + off + static_cast<size_t>(seg_num) * 4;
  if (workspace_bytes < need) return kInvalid;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = hipMemcpyAsync(h_status, reinterpret_cast<const void*>(ws + off),
                                static_cast<size_t>(seg_num) * 4, hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  return static_cast<int>(e);
}

}  // namespace
}  // namespace radix_topk_amd

using radix_topk_amd::kInfBitsBF16;
using radix_topk_amd::kInfBitsF16;

extern "C" {

size_t radix_topk_batch_topk_half_workspace_size(int seg_num, int seg_len, int k) {
  return radix_topk_amd::fixed_workspace_size(seg_num, seg_len, k);
}

int radix_topk_batch_topk_half(const uint16_t* d_input, int seg_num, int seg_len, int k,
                               uint16_t* d_output_values, int32_t* d_output_indices,
                               void* d_workspace, size_t workspace_bytes, void* stream) {
  return radix_topk_amd::fixed_topk(kInfBitsF16, d_input, seg_num, seg_len, k, d_output_values,
                                    d_output_indices, d_workspace, workspace_bytes, stream);
}

size_t radix_topk_batch_topk_half_segmented_workspace_size(int seg_num, int max_seg_len, int k) {
  return radix_topk_amd::segmented_workspace_size(seg_num, max_seg_len, k);
}

int radix_topk_batch_topk_half_segmented(const uint16_t* d_input, const int32_t* d_offsets,
                                         int seg_num, int max_seg_len, int k,
                                         uint16_t* d_output_values, int32_t* d_output_indices,
                                         void* d_workspace, size_t workspace_bytes,
                                         void* stream) {
  return radix_topk_amd::segmented_topk(kInfBitsF16, d_input, d_offsets, seg_num, max_seg_len, k,
                                        d_output_values, d_output_indices, d_workspace,
                                        workspace_bytes, stream);
}

size_t radix_topk_batch_topk_bf16_workspace_size(int seg_num, int seg_len, int k) {
  return radix_topk_amd::fixed_workspace_size(seg_num, seg_len, k);
}

int radix_topk_batch_topk_bf16(const uint16_t* d_input, int seg_num, int seg_len, int k,
                               uint16_t* d_output_values, int32_t* d_output_indices,
                               void* d_workspace, size_t workspace_bytes, void* stream) {
  return radix_topk_amd::fixed_topk(kInfBitsBF16, d_input, seg_num, seg_len, k, d_output_values,
                                    d_output_indices, d_workspace, workspace_bytes, stream);
}

size_t radix_topk_batch_topk_bf16_segmented_workspace_size(int seg_num, int max_seg_len, int k) {
  return radix_topk_amd::segmented_workspace_size(seg_num, max_seg_len, k);
}

int radix_topk_batch_topk_bf16_segmented(const uint16_t* d_input, const int32_t* d_offsets,
                                         int seg_num, int max_seg_len, int k,
                                         uint16_t* d_output_values, int32_t* d_output_indices,
                                         void* d_workspace, size_t workspace_bytes,
                                         void* stream) {
  return radix_topk_amd::segmented_topk(kInfBitsBF16, d_input, d_offsets, seg_num, max_seg_len, k,
                                        d_output_values, d_output_indices, d_workspace,
                                        workspace_bytes, stream);
}

size_t radix_topk_batch_topk_f32_workspace_size(int seg_num, int seg_len, int k) {
  return radix_topk_amd::fixed_workspace_size(seg_num, seg_len, k, radix_topk_amd::kInfBitsF32);
}

int radix_topk_batch_topk_f32(const float* d_input, int seg_num, int seg_len, int k, float* d_output_values,
                              int32_t* d_output_indices, void* d_workspace, size_t workspace_bytes,
                              void* stream) {
  return radix_topk_amd::fixed_topk(radix_topk_amd::kInfBitsF32, d_input, seg_num, seg_len, k,
                                    d_output_values, d_output_indices, d_workspace, workspace_bytes,
                                    stream);
}

size_t radix_topk_batch_topk_f32_segmented_workspace_size(int seg_num, int max_seg_len, int k) {
  return radix_topk_amd::segmented_workspace_size(seg_num, max_seg_len, k, radix_topk_amd::kInfBitsF32);
}

int radix_topk_batch_topk_f32_segmented(const float* d_input, const int32_t* d_offsets, int seg_num,
                                        int max_seg_len, int k, float* d_output_values,
                                        int32_t* d_output_indices, void* d_workspace,
                                        size_t workspace_bytes, void* stream) {
  return radix_topk_amd::segmented_topk(radix_topk_amd::kInfBitsF32, d_input, d_offsets, seg_num,
                                        max_seg_len, k, d_output_values, d_output_indices, d_workspace,
                                        workspace_bytes, stream);
}

size_t radix_topk_batch_topk_ex_workspace_size(int format, int segmented, int seg_num, int seg_len,
                                               int k) {
  return radix_topk_amd::ex_workspace_size(format, segmented, seg_num, seg_len, k);
}

int radix_topk_batch_topk_ex(const void* d_input, int format, const int32_t* d_offsets, int seg_num,
                             int seg_len, int k, int flags, void* d_output_values,
                             int32_t* d_output_indices, void* d_workspace, size_t workspace_bytes,
                             void* stream) {
  return radix_topk_amd::topk_ex(d_input, format, d_offsets, seg_num, seg_len, k, flags, d_output_values,
                                 d_output_indices, d_workspace, workspace_bytes, stream);
}

size_t radix_topk_sample_half_workspace_size(int seg_num, int seg_len, int k) {
  return radix_topk_amd::fixed_workspace_size(seg_num, seg_len, k);
}

int radix_topk_sample_half(const uint16_t* d_logits, int seg_num, int seg_len, int k,
                           float temperature, const float* d_uniforms, uint16_t* d_topk_values,
                           int32_t* d_topk_indices, float* d_probs, int32_t* d_samples,
                           void* d_workspace, size_t workspace_bytes, void* stream) {
  return radix_topk_amd::sample_topk(false, d_logits, seg_num, seg_len, k, temperature, d_uniforms,
                                     d_topk_values, d_topk_indices, d_probs, d_samples, d_workspace,
                                     workspace_bytes, stream);
}

size_t radix_topk_sample_bf16_workspace_size(int seg_num, int seg_len, int k) {
  return radix_topk_amd::fixed_workspace_size(seg_num, seg_len, k);
}

int radix_topk_sample_bf16(const uint16_t* d_logits, int seg_num, int seg_len, int k,
                           float temperature, const float* d_uniforms, uint16_t* d_topk_values,
                           int32_t* d_topk_indices, float* d_probs, int32_t* d_samples,
                           void* d_workspace, size_t workspace_bytes, void* stream) {
  return radix_topk_amd::sample_topk(true, d_logits, seg_num, seg_len, k, temperature, d_uniforms,
                                     d_topk_values, d_topk_indices, d_probs, d_samples, d_workspace,
                                     workspace_bytes, stream);
}

int radix_topk_workspace_status(const void* d_workspace, size_t workspace_bytes, int seg_num,
                                uint32_t* h_status, void* stream) {
  return radix_topk_amd::workspace_status(d_workspace, workspace_bytes, seg_num, h_status, stream);
}

void radix_topk_debug_wait_hook(uint32_t spin_limit, uint32_t force_mask) {
  radix_topk_amd::g_wait_hook.store(
      spin_limit == 0 ? 0 : ((static_cast<uint64_t>(spin_limit) << 32) | force_mask), std::memory_order_relaxed);
}

}  // extern "C"
