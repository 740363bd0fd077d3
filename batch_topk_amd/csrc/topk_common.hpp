// Shared host/device definitions of the batched fp16 top-k engine.
#pragma once

#include <cstddef>
#include <cstdint>

namespace radix_topk_amd {

// Largest k of every entry point (RADIX_TOPK_MAX_K of the C ABI).
constexpr int kMaxTopK = 1024;

// LDS entries (8 bytes each) of a workgroup's candidate area: the per-wave candidate regions,
// then the contiguous candidate list, and for a multi-workgroup segment the merged lists.
constexpr int kCandArea = 2048;
// Per-wave private LDS region of the filter, in 32-bit words (kStageWords / 2 candidates).
constexpr int kStageWords = 512;
// Longest chunk one workgroup covers: 1024 threads x 16 vectors x 8 elements.
constexpr int kMaxChunk = 1024 * 16 * 8;

// Cooperative (whole-segment threshold) path: per-segment workspace block of a segment split
// over W workgroups.  Nothing in it needs clearing before a call except the histograms, which
// workgroup 0 clears at the start of the call.  Every word one workgroup writes for another
// carries a per-call token derived from the host's call epoch and the block's generation
// word, which the call advances, so a replayed call (same epoch) never takes a word left by an
// earlier replay for its own:
//   flag    u64                       "histograms cleared" word (tag44 << 20 | 1), and at
//                                     byte 8 the generation word (read by every workgroup at
//                                     its start, advanced once all have read it)
//   arrive  u64 [kGroupBarriers][W]   per-barrier arrival slots (a slot holding this call's
//                                     token has arrived)
//   counts  u64 [2][W]                epoch-tagged list lengths (tag44 << 20 | length)
//   hist    u32 [kGroupCopies][256]   threshold histogram of the thread bests' high key byte,
//                                     spread over kGroupCopies copies so that few workgroups
//                                     add to one address
//   fine    u32 [kFineCopies][2048]   the same thread bests at 32-key resolution (key >> 5)
//   rhist   u32 [kRefineDigits][256]  refinement digit histograms (6 digits of a 16-bit key and
//                                     a 32-bit index, 8 with a 32-bit key)
//   lists   u64 [W][kCandArea]        every workgroup's candidate list
constexpr int kRefineDigits = 8;
constexpr int kGroupBarriers = 3 + kRefineDigits;
constexpr int kGroupCopies = 4;
constexpr int kFineCopies = 4;
constexpr int kFineBins = 2048;
// Longest whole-segment list the final ranking takes: it is gathered into the LDS from the
// candidate area onward (area, selection, rank and staging regions, free by then), which
// holds at least 6464 entries for every k.
constexpr int kGroupCap = 6144;
struct GroupLayout {
  size_t flag, arrive, counts, hist, fine, rhist, lists, bytes;
};
constexpr size_t group_align(size_t x) { return (x + 127) / 128 * 128; }
constexpr GroupLayout group_layout(int W) {
  GroupLayout L{};
  size_t off = 0;
  L.flag = off;
  off += 128;
  L.arrive = off;
  off += group_align(static_cast<size_t>(kGroupBarriers) * W * 8);
  L.counts = off;
  off += group_align(static_cast<size_t>(2) * W * 8);
  L.hist = off;
  off += static_cast<size_t>(kGroupCopies) * 256 * 4;
  L.fine = off;
  off += static_cast<size_t>(kFineCopies) * kFineBins * 4;
  L.rhist = off;
  off += static_cast<size_t>(kRefineDigits) * 256 * 4;
  L.lists = off;
  off += static_cast<size_t>(W) * kCandArea * 8;
  L.bytes = off;
  return L;
}
// Most co-resident workgroups the cooperative path asks for (one 1024-thread workgroup per CU
// of an MI355X).
constexpr int kMaxCoopGroups = 256;

// Per-segment completion status (one u32 per segment in the workspace, written by every call;
// RADIX_TOPK_STATUS_* of the C ABI).  A cross-workgroup wait is bounded: a workgroup that
// gives up on one (its peers were not resident, or a test forced it) records kStatusTimeout
// and fills its segment's row with the pad instead of hanging.
constexpr uint32_t kStatusOk = 0;
constexpr uint32_t kStatusTimeout = 1;
// Polls of every bounded cross-workgroup wait (each poll is a device-coherent load and a
// short sleep): about a second, far beyond any wait between co-resident workgroups.
constexpr uint32_t kDefaultSpinLimit = 1u << 22;
// Test hook bits (TopkParams::force_timeout): the named wait looks for a value nobody writes,
// so it runs to its spin limit and takes the give-up path.
constexpr uint32_t kForceFlagWait = 1;      // cooperative "histograms cleared" wait
constexpr uint32_t kForceBarrier = 2;       // cooperative first barrier
constexpr uint32_t kForceCollect = 4;       // cooperative list-length collection
constexpr uint32_t kForcePairPoll = 8;      // two-chunk merger's poll for the published list

// +inf bit patterns of the two 16-bit element formats; a magnitude above it is a NaN.
constexpr uint32_t kInfBitsF16 = 0x7C00u;
constexpr uint32_t kInfBitsBF16 = 0x7F80u;
// +inf of fp32; passed as the format tag of the 32-bit element path.
constexpr uint32_t kInfBitsF32 = 0x7F800000u;

// Kernel parameter block of the fused segmented top-k kernel.  Every segment s covers the
// element range [s0, s1) of `base` (a 16-byte aligned pointer); s0/s1 come from the int32
// offsets when given, else from s * seg_len.  `elem0` is the element offset of the caller's
// input pointer from `base` (0..7), added to every segment bound.
struct TopkParams {
  const uint16_t* base;
  const int32_t* offsets;       // device [seg_num + 1] or nullptr (fixed-length segments)
  int64_t elem0;
  int64_t seg_len;              // fixed-length mode only
  int64_t max_len;              // longest segment the launch covers; longer rows are padded
  int32_t seg_num;
  int32_t k;
  int32_t chunks_per_seg;       // W: workgroups per segment; grid.x = seg_num * W
  int32_t cap_chunk;            // LDS capacity of one chunk's candidate list
  int32_t cap_list;             // workspace capacity of one chunk's published list
  int32_t cand_area;            // LDS entries of the candidate / merge area
  int32_t kpad;                 // LDS entries of the selection area (power of two >= k)
  int32_t cooperative;          // 1: whole-segment threshold across the segment's workgroups
  void* out_vals;               // [seg_num, k] element bits (2 or 4 bytes), or nullptr: indices only
  int32_t unsorted;             // 1: each row's selected set in unspecified order
  int32_t* out_idx;             // [seg_num, k]
  unsigned long long* tickets;  // [seg_num] arrival words (epoch << 16 | count)
  int32_t* list_counts;         // [seg_num * W]
  unsigned long long* lists;    // [seg_num * W * cap_list] packed (key16 << 32 | index)
  unsigned long long epoch;     // 48-bit token unique to this call
  uint32_t inf_bits;            // +inf pattern of a 16-bit element format (0x7C00 fp16, 0x7F80 bf16)
  int32_t elem_bytes;           // 2 (fp16, bf16) or 4 (fp32)
  // Top-k sampling fused into the last step (non-cooperative plans), off when samples is null.
  const float* uniforms;        // [seg_num] u in [0, 1)
  int32_t* samples;             // [seg_num] sampled index (-1 for an empty segment)
  float* probs;                 // [seg_num, k] or nullptr
  float inv_temperature;        // 1 / temperature, rounded to fp32
  unsigned char* groups;        // cooperative path: [seg_num] blocks of group_layout(W).bytes
  int32_t group;                // long-segment path: workgroups per segment (each takes every
                                //   group-th chunk of it), 0 on every other path
  uint32_t* status;             // [seg_num] completion status of this call (kStatus*)
  uint32_t spin_limit;          // polls of every bounded cross-workgroup wait
  uint32_t force_timeout;       // test hook: kForce* bits (0 in every ordinary call)
};

// One compiled instantiation of the fused kernel.
struct KernelShape {
  int block;  // threads per workgroup (multiple of 64)
  int vpt;    // 16-byte vectors per thread
};

// Launch plan: everything the host derives from (seg_num, max segment length, k).
struct Plan {
  KernelShape shape;
  int chunk;        // elements per workgroup = block * vpt * 8
  int W;            // workgroups per segment
  int cap_chunk;
  int cap_list;
  int cand_area;
  int kpad;
  size_t lds_bytes;
  size_t ws_bytes;  // workspace bytes (includes 256 bytes of alignment slack)
  bool cooperative; // all W workgroups of a segment co-resident, one shared threshold
  int group;        // long-segment path (> 0): workgroups per segment, each taking several
                    // chunks; the grid is seg_num * group (co-resident when group > 1)
  bool ok;
};

// Device launch of the fused kernel for `plan` (implemented in topk_kernels.hip).
int launch_segmented_topk(const Plan& plan, const TopkParams& params, void* stream);

// Parameter block of the sampling kernel (sample_kernels.hip): one draw per row from the
// softmax of the row's top-k values (already written by the top-k kernel, in rank order).
struct SampleParams {
  const uint16_t* topk_vals;  // [seg_num, k] raw 16-bit values in rank order
  const int32_t* topk_idx;    // [seg_num, k] indices; -1 marks ranks past a short segment
  const float* uniforms;      // [seg_num] u in [0, 1)
  int32_t* samples;           // [seg_num] sampled index (-1 for an empty segment)
  float* probs;               // [seg_num, k] or nullptr
  float inv_temperature;      // 1 / temperature, rounded to fp32
  int32_t seg_num;
  int32_t k;
  int32_t bf16;               // 1: values are bfloat16 bits, 0: fp16
};

// Device launch of the sampling kernel (implemented in sample_kernels.hip).
int launch_topk_sample(const SampleParams& params, void* stream);

}  // namespace radix_topk_amd
