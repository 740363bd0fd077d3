/*
 * batch_topk for AMD Instinct MI355X (gfx950) -- C ABI.
 *
 * Batched fp16 top-k with int32 index output.  For every segment the k best values are
 * returned in descending order together with their segment-local indices.  The order
 * is total and deterministic: larger value first, equal values by ascending index, every
 * NaN (any sign or payload) below -inf, and +0 equal to -0.  Output values are the raw
 * 16-bit patterns read from the input at the selected index (NaN payloads and the sign
 * of zero are preserved).
 *
 * All pointers named d_* are device pointers (hipMalloc'd or equivalent).  fp16 data
 * travels as uint16_t bit patterns so that plain C and FFI callers need no half type;
 * the memory layout is identical to __half.  `stream` is a hipStream_t (NULL = the
 * null stream).  Every call is stream-ordered and asynchronous; nothing is allocated
 * and the host never synchronises.
 *
 * Return values are hipError_t codes as int: 0 = hipSuccess; 1 = hipErrorInvalidValue
 * for any rejected argument, returned before any HIP call is made; otherwise the HIP
 * error of the failed launch.  Long segments with large k run as one cooperative grid
 * whose workgroups must all be resident at once (one per CU); a shape that needs more
 * workgroups than the device has CUs returns hipErrorCooperativeLaunchTooLarge.
 *
 * The workspace is owned by the caller, its content on entry may be arbitrary, and it
 * must not be shared by calls that can run concurrently.
 */
#ifndef BATCH_TOPK_AMD_BATCH_TOPK_H_
#define BATCH_TOPK_AMD_BATCH_TOPK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Largest k accepted by every entry point. */
#define RADIX_TOPK_MAX_K 1024

/*
 * Fixed-length segments: segment s is d_input[s*seg_len, (s+1)*seg_len).
 * Outputs are [seg_num, k] row-major.
 *
 * Replaces radix_topk::batch_topk_half (reference include/batch_topk.cuh:10-19,
 * implemented at src/batch_topk.cu:42-193) with the same argument order and meaning.
 * Rejected (-> 1): seg_num <= 0, seg_len <= 0, k <= 0, k > seg_len, k > RADIX_TOPK_MAX_K,
 * any NULL pointer, workspace_bytes below the size reported by
 * radix_topk_batch_topk_half_workspace_size (reference src/batch_topk.cu:13-33).
 */
int radix_topk_batch_topk_half(const uint16_t* d_input, int seg_num, int seg_len, int k,
                               uint16_t* d_output_values, int32_t* d_output_indices,
                               void* d_workspace, size_t workspace_bytes, void* stream);

/*
 * Workspace bytes for radix_topk_batch_topk_half; 0 for an unsupported shape.
 * Replaces radix_topk::batch_topk_half_workspace_size (reference include/batch_topk.cuh:21,
 * src/batch_topk.cu:35-40).  Depends only on the shape, never on the data or the device.
 */
size_t radix_topk_batch_topk_half_workspace_size(int seg_num, int seg_len, int k);

/*
 * Variable-length segments: segment s is d_input[d_offsets[s], d_offsets[s+1]),
 * d_offsets being a device int32 array of seg_num + 1 non-decreasing entries.
 * max_seg_len is a host-known upper bound on every segment length and sizes the launch.
 * Segments shorter than k (including empty ones) fill ranks >= length with index -1 and
 * value bits 0xFFFF.  A segment longer than max_seg_len breaks the precondition: its
 * whole output row is filled with that pad.
 *
 * No counterpart in the reference, which has fixed-length segments only; it extends
 * radix_topk::batch_topk_half (reference include/batch_topk.cuh:10-19) with the offset
 * array used by segmented callers.
 * Rejected (-> 1): seg_num <= 0, max_seg_len < 0, k <= 0, k > RADIX_TOPK_MAX_K, any NULL
 * pointer, workspace_bytes below radix_topk_batch_topk_half_segmented_workspace_size.
 */
int radix_topk_batch_topk_half_segmented(const uint16_t* d_input, const int32_t* d_offsets,
                                         int seg_num, int max_seg_len, int k,
                                         uint16_t* d_output_values, int32_t* d_output_indices,
                                         void* d_workspace, size_t workspace_bytes,
                                         void* stream);

/*
 * Workspace bytes for radix_topk_batch_topk_half_segmented; 0 for an unsupported shape.
 * Extends radix_topk::batch_topk_half_workspace_size (reference include/batch_topk.cuh:21)
 * to the segmented entry point.
 */
size_t radix_topk_batch_topk_half_segmented_workspace_size(int seg_num, int max_seg_len, int k);

/*
 * bfloat16 twins of the four entry points above: the same arguments, contract, workspace
 * sizes and error behaviour, for segments of bfloat16 bit patterns.  The order is the same
 * total order (larger value first, equal values by ascending index, every NaN below -inf,
 * +0 equal to -0), with bfloat16's own inf/NaN boundary (exponent all ones).  No
 * counterpart in the reference, whose codec covers fp16 only (reference
 * include/type_codec.cuh:9-38); bfloat16 widens exactly to float, so the reference's
 * verifier order (include/batch_topk_types.cuh:70-82) applies to it unchanged.
 */
int radix_topk_batch_topk_bf16(const uint16_t* d_input, int seg_num, int seg_len, int k,
                               uint16_t* d_output_values, int32_t* d_output_indices,
                               void* d_workspace, size_t workspace_bytes, void* stream);
size_t radix_topk_batch_topk_bf16_workspace_size(int seg_num, int seg_len, int k);
int radix_topk_batch_topk_bf16_segmented(const uint16_t* d_input, const int32_t* d_offsets,
                                         int seg_num, int max_seg_len, int k,
                                         uint16_t* d_output_values, int32_t* d_output_indices,
                                         void* d_workspace, size_t workspace_bytes,
                                         void* stream);
size_t radix_topk_batch_topk_bf16_segmented_workspace_size(int seg_num, int max_seg_len, int k);

/*
 * Top-k sampling (LLM decoding): the top-k of every row exactly as radix_topk_batch_topk_half
 * (written to d_topk_values / d_topk_indices), then one index drawn per row from the softmax
 * of its top-k at the given temperature, using the caller's uniform d_uniforms[row] in [0, 1).
 * With v_0 >= v_1 >= ... the row's top-k values in output order (as floats) and m the number
 * of ranks with an index >= 0:
 *   w_0 = 1; for r >= 1, w_r = 1 if v_r == v_0, else exp((v_r - v_0) * (1 / temperature))
 *   (1 / temperature rounded to float), and 0 where that is NaN;
 *   S = w_0 + ... + w_{m-1};  d_samples[row] = the index at the first rank r whose running
 *   sum w_0 + ... + w_r exceeds u * S (the last rank if rounding leaves none);
 *   d_probs[row * k + r] = w_r / S (0 past m), when d_probs is not NULL.
 * Sums are in fp32, so probabilities carry fp32 rounding; the top-k itself is bit-exact.
 * Rejected (-> 1): everything batch_topk_half rejects, temperature not finite or <= 0,
 * NULL d_uniforms or d_samples.  Workspace: radix_topk_sample_half_workspace_size (equal to
 * the top-k's).  Two launches on `stream`, nothing allocated.
 * No counterpart in the reference; it is the consumer the reference's LLM-sampling workload
 * (128 x 128,256 logits, k = 50) feeds.
 */
int radix_topk_sample_half(const uint16_t* d_logits, int seg_num, int seg_len, int k,
                           float temperature, const float* d_uniforms, uint16_t* d_topk_values,
                           int32_t* d_topk_indices, float* d_probs, int32_t* d_samples,
                           void* d_workspace, size_t workspace_bytes, void* stream);
size_t radix_topk_sample_half_workspace_size(int seg_num, int seg_len, int k);
/* The same for bfloat16 logits (top-k as radix_topk_batch_topk_bf16). */
int radix_topk_sample_bf16(const uint16_t* d_logits, int seg_num, int seg_len, int k,
                           float temperature, const float* d_uniforms, uint16_t* d_topk_values,
                           int32_t* d_topk_indices, float* d_probs, int32_t* d_samples,
                           void* d_workspace, size_t workspace_bytes, void* stream);
size_t radix_topk_sample_bf16_workspace_size(int seg_num, int seg_len, int k);

/*
 * fp32 twins of the four fixed-length and segmented entry points: the same arguments,
 * contract and error behaviour, for float input and float output values (the raw 32-bit
 * patterns of the selected elements, NaN payloads and the sign of zero preserved; pads are
 * index -1 with bits 0xFFFFFFFF).  The order is the reference verifier's own, which compares
 * floats (reference include/batch_topk_types.cuh:70-82): larger first, ties by ascending
 * index, every NaN below -inf, +0 equal to -0.  Pointers must be 4-byte aligned.  Workspace
 * sizes are their own (four elements per 16-byte load instead of eight); a segment needing
 * more cooperative workgroups than an MI355X has CUs (k large and more than 16.7 M floats)
 * is unsupported (size 0).  No counterpart in the reference, whose codec covers fp16 only.
 */
int radix_topk_batch_topk_f32(const float* d_input, int seg_num, int seg_len, int k,
                              float* d_output_values, int32_t* d_output_indices,
                              void* d_workspace, size_t workspace_bytes, void* stream);
size_t radix_topk_batch_topk_f32_workspace_size(int seg_num, int seg_len, int k);
int radix_topk_batch_topk_f32_segmented(const float* d_input, const int32_t* d_offsets,
                                        int seg_num, int max_seg_len, int k,
                                        float* d_output_values, int32_t* d_output_indices,
                                        void* d_workspace, size_t workspace_bytes, void* stream);
size_t radix_topk_batch_topk_f32_segmented_workspace_size(int seg_num, int max_seg_len, int k);

/* Element formats and output flags of radix_topk_batch_topk_ex. */
#define RADIX_TOPK_FORMAT_F16 0  /* IEEE binary16 bit patterns */
#define RADIX_TOPK_FORMAT_BF16 1 /* bfloat16 bit patterns */
#define RADIX_TOPK_FORMAT_F32 2  /* IEEE binary32 (float); values are 4 bytes */
#define RADIX_TOPK_UNSORTED 1     /* each row's selected entries in unspecified order */
#define RADIX_TOPK_INDICES_ONLY 2 /* no values: d_output_values may be NULL and is not written */

/*
 * One entry point for every input layout, element format and output variant.
 *   d_offsets == NULL: fixed-length segments of seg_len elements, as
 *     radix_topk_batch_topk_half / _bf16 (including k <= seg_len);
 *   d_offsets != NULL: variable-length segments with seg_len the host-known maximum length,
 *     as radix_topk_batch_topk_half_segmented / _bf16_segmented.
 * flags = 0 gives exactly those entry points' results.  RADIX_TOPK_UNSORTED keeps each
 * row's first min(k, length) slots as the same set of (index, value) entries, in an order
 * that is unspecified and may differ between calls; the slots past them hold the pad.
 * It saves the rank counting of long candidate lists.  RADIX_TOPK_INDICES_ONLY writes only
 * the indices (2 bytes less per output rank).
 * Rejected (-> 1): an unknown format or flag, NULL d_output_values without
 * RADIX_TOPK_INDICES_ONLY, and everything the fixed-length or segmented entry point of the
 * same layout rejects.
 * No counterpart in the reference, which always writes sorted values and indices
 * (reference include/batch_topk.cuh:10-19); unsorted and indices-only outputs serve callers
 * that need neither the order nor the values (a sampler over indices, a set membership).
 */
int radix_topk_batch_topk_ex(const void* d_input, int format, const int32_t* d_offsets, int seg_num,
                             int seg_len, int k, int flags, void* d_output_values,
                             int32_t* d_output_indices, void* d_workspace, size_t workspace_bytes,
                             void* stream);
/* Workspace bytes for radix_topk_batch_topk_ex (segmented != 0: d_offsets given); 0 for an
 * unsupported shape or format.  Equal to the size of the matching fixed-length or segmented
 * entry point. */
size_t radix_topk_batch_topk_ex_workspace_size(int format, int segmented, int seg_num, int seg_len,
                                               int k);

/*
 * Allocation-free twin of radix_topk_batch_topk_half, for callers that cannot allocate device
 * memory or pass a workspace (code under HIP-graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The same arguments without the workspace, the same results and the same
 * rejections (1 = hipErrorInvalidValue before any HIP call); the workspace is instead a static
 * device array of RADIX_TOPK_NOALLOC_SCRATCH_BYTES bytes, one per GPU, held until the process
 * ends.  A shape whose workspace (radix_topk_batch_topk_half_workspace_size) exceeds it returns
 * 2 (hipErrorOutOfMemory) before any HIP call.  Nothing is allocated: the first call on a
 * device looks up the array's address (hipGetSymbolAddress) and keeps it.  Every call on one
 * GPU uses the same array, so calls that can overlap on one GPU (different streams, other
 * host threads) race and must not be issued concurrently; calls in one stream are ordered.
 * No counterpart in the reference, whose callers always pass a workspace
 * (reference include/batch_topk.cuh:10-19).
 */
#define RADIX_TOPK_NOALLOC_SCRATCH_BYTES (8u << 20)
int radix_topk_batch_topk_half_noalloc(const uint16_t* d_input, int seg_num, int seg_len, int k,
                                       uint16_t* d_output_values, int32_t* d_output_indices,
                                       void* stream);

/* Per-segment completion status of a call (radix_topk_workspace_status). */
#define RADIX_TOPK_STATUS_OK 0
#define RADIX_TOPK_STATUS_WAIT_TIMEOUT 1

/*
 * Completion status of the last call made with this workspace, one word per segment, copied
 * to the host array h_status[seg_num] (seg_num as in that call).  The call synchronises
 * `stream`, on which the top-k call must have been issued (or a stream ordered after it).
 *   RADIX_TOPK_STATUS_OK: the segment's row was written completely.
 *   RADIX_TOPK_STATUS_WAIT_TIMEOUT: a workgroup of the segment gave up a bounded wait for
 *   another workgroup of the same call (the segment's workgroups were not all resident at
 *   once, e.g. because kernels of other streams or processes held the GPU's compute units);
 *   the row holds the pad (index -1, value bits all ones) in some or all ranks.
 * Segments split over several workgroups wait for each other: long segments with large k run
 * as one grid whose workgroups must all be resident at once.  Every such wait is bounded, so
 * the kernel always finishes; this query tells a caller whether the rows are complete.
 * Every call rewrites every segment's word, so a call after a timed-out one reports its own
 * status.  Returns 0, 1 (NULL pointers, seg_num <= 0, workspace too small for seg_num
 * segments) or the HIP error of the copy.
 * No counterpart in the reference, whose chain of kernel launches never waits across
 * workgroups (reference src/batch_topk.cu:42-193).
 */
int radix_topk_workspace_status(const void* d_workspace, size_t workspace_bytes, int seg_num,
                                uint32_t* h_status, void* stream);

/*
 * Test hook, not for production use: every later call bounds each cross-workgroup wait at
 * spin_limit polls and, for every bit of force_mask (1: the long-segment grid's first wait,
 * 2: its first meeting, 4: its list collection, 8: the two-chunk merge), makes that wait look
 * for a value no workgroup writes, so it times out, fills the segment's row with the pad and
 * reports RADIX_TOPK_STATUS_WAIT_TIMEOUT, with every kernel still running to its end.
 * spin_limit = 0 restores ordinary calls.  Process-wide; not synchronised with calls in flight.
 */
void radix_topk_debug_wait_hook(uint32_t spin_limit, uint32_t force_mask);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* BATCH_TOPK_AMD_BATCH_TOPK_H_ */
