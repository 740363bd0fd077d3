// Fused segmented top-k for gfx950 (MI355X): fp16 and bf16 (16-bit elements) and fp32.
//
// One workgroup owns one chunk (block * vpt * 8 16-bit elements, or * 4 floats) of one
// segment; a segment of up to 131,072 16-bit elements is a single chunk.  The steps below are
// written for 16-bit elements; for fp32 they run on the top 16 bits of the 32-bit key, and
// the candidates carry the exact key (see Elem16 / Elem32).  The chunk is read from HBM exactly once, with
// nontemporal 16-byte loads that are all issued up front, into registers.  Everything after
// the load runs on registers and LDS, overlapped with the loads still in flight:
//
//   1. thread best     packed int16 max/min trees over the raw fp16 bits of all the thread's
//                      vectors (v_pk_max_i16 / v_pk_min_i16).  The int16 max is the best
//                      non-negative-sign element, the int16 min the best negative-sign one;
//                      whichever applies is a real element of the thread (or, for a NaN, a
//                      worse one), which is all the threshold needs.
//   2. threshold       T = the kc-th smallest descending key among the thread bests, found
//                      exactly with two LDS histogram passes (high byte, then low byte inside
//                      the boundary bucket) and DPP prefix scans.  At least kc real elements
//                      have key <= T, so every element of the chunk's top kc does.
//   3. filter          only a vector whose int16 max reaches T can hold a candidate.  A wave
//                      copies its lanes' passing vectors into an LDS staging list and tests
//                      them one vector per lane; a wave prefix sum places the hits, which one
//                      LDS atomic per wave reserves in the list, packed as
//                      (key16 << 48 | index32 << 16 | raw16): one u64 compare orders
//                      (key, index), and the raw bits ride along to the output.
//                      If the list overflows (ties, all-equal rows), an exact radix refinement
//                      over (key16, position17), re-reading the chunk, rebuilds it.
//   4. selection       small sets: every candidate counts the entries below it (one DPP row
//                      per candidate up to 128; up to 32 entries per wave, one lane per
//                      candidate over 16-byte LDS broadcasts); larger sets: LDS radix select
//                      over the packed values down to exactly k, then rank counting.
//   5. output          index and raw value bits of each selected candidate.
//
// Segments longer than one chunk are split over W workgroups.  While the W lists fit one LDS
// merge, they meet once through the workspace, which needs no initialisation.  Two chunks:
// the workgroup that takes the segment's ticket first (an exchange issued while its loads are
// in flight) publishes its list with every word tagged for the call, and the other polls for
// it and merges it with its own list in step 4.  Three or more: each workgroup publishes, and
// the last to arrive (an epoch-tagged arrival counter) merges.  Beyond that (long segments with large k) the W workgroups run cooperatively, all
// co-resident: the threshold histograms of step 2 are summed over the whole segment in global
// memory, each workgroup filters its chunk against the one segment threshold, and every
// workgroup gathers the segment's candidate list and ranks a share of it.  Workgroups meet at
// barriers made of per-workgroup arrival slots holding the call's epoch; an exact global
// radix refinement over (key16, index32) takes over when the list would not fit.
//
// Ordering contract (reference include/batch_topk_types.cuh:70-82,100-113 and
// include/type_codec.cuh:9-38): ascending (desc_key, index), where desc_key maps every NaN
// to 0xFFFF, +-0 to 0x7FFF, and is strictly decreasing in value otherwise.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <type_traits>

#include "sample_row.hpp"
#include "topk_common.hpp"

// Phase timestamps, compiled only into the profiling build (-DTOPK_PHASE_TRACE, a library of
// its own that batch_topk_amd.profiling loads); in the engine every hook is empty.
//   TOPK_TRACE(id): thread 0 of workgroup b stores the shader clock (s_memtime) and the
//     constant 100 MHz clock (s_memrealtime) in slot id of row b; id 0 also clears the row.
//   TOPK_WTRACE(id): lane 0 of every wave stores the shader clock in slot id of its wave's row.
//   TOPK_TRACE_VALUE(id, v): thread 0 stores v in slot id of row b (shader-clock table).
// Slots: 0 start, 12 loads issued, 1 thread best, 2 first histogram round, 4 threshold,
// 5 filter, 6 refinement done, 8 first meeting (cooperative) or list published (two-chunk
// segment), 9 cooperative threshold, 10 list stored or lists merged, 3 cooperative lengths
// read, 7 cooperative lists gathered, 11 end; values: 13 merger's poll rounds, 14 candidates,
// 15 threshold.  Wave slots: 1 thread best, 0 threshold read, 2 filter start, 3 vectors
// staged, 4 flushed, 5 after the filter barrier, 6 ranking start, 7 ranking end.
#ifdef TOPK_PHASE_TRACE
namespace radix_topk_amd_trace {
constexpr int kMaxWorkgroups = 2048;
__device__ unsigned long long g_clock[kMaxWorkgroups * 16];
__device__ unsigned long long g_real[kMaxWorkgroups * 16];
__device__ unsigned long long g_wave[kMaxWorkgroups * 16 * 16];
}  // namespace radix_topk_amd_trace
#define TOPK_TRACE(id)                                                                         \
  do {                                                                                         \
    if (threadIdx.x == 0 && blockIdx.x < radix_topk_amd_trace::kMaxWorkgroups) {               \
      unsigned long long* row_ = radix_topk_amd_trace::g_clock + blockIdx.x * 16;              \
      unsigned long long* real_ = radix_topk_amd_trace::g_real + blockIdx.x * 16;              \
      if ((id) == 0)                                                                           \
        for (int q_ = 1; q_ < 16; ++q_) row_[q_] = real_[q_] = 0;                              \
      row_[(id)] = __builtin_amdgcn_s_memtime();                                               \
      real_[(id)] = __builtin_amdgcn_s_memrealtime();                                          \
    }                                                                                          \
  } while (0)
#define TOPK_WTRACE(id)                                                                        \
  do {                                                                                         \
    if ((threadIdx.x & 63) == 0 && blockIdx.x < radix_topk_amd_trace::kMaxWorkgroups)          \
      radix_topk_amd_trace::g_wave[(blockIdx.x * 16 + (threadIdx.x >> 6)) * 16 + (id)] =       \
          __builtin_amdgcn_s_memtime();                                                        \
  } while (0)
#define TOPK_TRACE_VALUE(id, value)                                                            \
  do {                                                                                         \
    if (threadIdx.x == 0 && blockIdx.x < radix_topk_amd_trace::kMaxWorkgroups)                 \
      radix_topk_amd_trace::g_clock[blockIdx.x * 16 + (id)] = (value);                         \
  } while (0)
#else
#define TOPK_TRACE(id)
#define TOPK_WTRACE(id)
#define TOPK_TRACE_VALUE(id, value)
#endif

namespace radix_topk_amd {
namespace {

using u32 = uint32_t;
using u64 = unsigned long long;
typedef short short2_t __attribute__((ext_vector_type(2)));
typedef unsigned short ushort2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
// 32 words held in registers and read at a wave-uniform index (s_set_gpr_idx), so a loop over
// a data-dependent set of a lane's vectors compiles to one short body instead of one per vector.
typedef unsigned u32x32_t __attribute__((ext_vector_type(32)));

// Word 3 of a gfx9 buffer resource (raw, untyped: data format 32 bits) and the nontemporal
// cache policy of a buffer load.
constexpr int kBufferWord3 = 0x00020000;
constexpr int kCachePolicyNT = 2;
constexpr int kArea = kCandArea;        // LDS candidate entries (candidate list, merged lists)
constexpr int kRankCap = 512;           // rank-counting path handles up to this many
constexpr int kSortRankMin = 256;       // lists at least this long are ranked by sorted runs

// ------------------------------------------------------------------------------ codec

// Descending order-preserving key of raw 16-bit float bits (reference
// include/type_codec.cuh:13-38 for fp16): NaN -> 0xFFFF, +-0 -> 0x7FFF, negative -> bits,
// positive -> bits ^ 0x7FFF.  fp16 and bf16 are both sign-magnitude with an all-ones exponent
// for inf and NaN; `inf` is the format's +inf pattern (0x7C00 fp16, 0x7F80 bf16) and a
// magnitude above it is a NaN.
__device__ __forceinline__ u32 desc_key(u32 b, u32 inf) {
  const u32 mag = b & 0x7fffu;
  u32 key = (b & 0x8000u) ? b : (b ^ 0x7fffu);
  key = (mag == 0u) ? 0x7fffu : key;
  key = (mag > inf) ? 0xffffu : key;
  return key;
}

// Candidate packing: ascending u64 order == ascending (key, index); raw bits carried along.
__device__ __forceinline__ u64 pack_candidate(u32 raw, u32 index, u32 inf) {
  return (static_cast<u64>(desc_key(raw, inf)) << 48) | (static_cast<u64>(index) << 16) | raw;
}
__device__ __forceinline__ u32 cand_index(u64 P) { return static_cast<u32>(P >> 16); }
__device__ __forceinline__ u32 cand_raw(u64 P) { return static_cast<u32>(P) & 0xffffu; }

// The same key for raw fp32 bits: NaN -> 0xFFFFFFFF, +-0 -> 0x7FFFFFFF, negative -> bits,
// positive -> bits ^ 0x7FFFFFFF.
__device__ __forceinline__ u32 desc_key32(u32 b) {
  const u32 mag = b & 0x7fffffffu;
  u32 key = (b & 0x80000000u) ? b : (b ^ 0x7fffffffu);
  key = (mag == 0u) ? 0x7fffffffu : key;
  key = (mag > 0x7f800000u) ? 0xffffffffu : key;
  return key;
}

// Element formats.  The kernel is written once for 16-bit and 32-bit elements.  Thread bests,
// threshold histograms and the filter bound always work on 16-bit key prefixes; candidates
// carry the exact key, so the selection among them is exact.
//   Elem16 (fp16, bf16; the +inf pattern comes at run time): 8 elements per 16-byte vector,
//     candidate = key16 << 48 | index << 16 | raw16.
//   Elem32 (fp32): 4 elements per vector, candidate = key32 << 32 | index.  The top 16 bits
//     of the key order like the key, so every element of a row's top k passes a threshold on
//     them; the raw bits of an output entry are decoded from its key (re-read from the input
//     for +-0 and NaN, whose keys merge several patterns).
struct Elem16 {
  static constexpr int kPerVec = 8;
  static constexpr int kBytes = 2;
  static constexpr int kKeyBits = 16;
  static constexpr int kIdxShift = 16;  // index field of a candidate
  static constexpr int kLowDigit = 16;  // radix digits below this never tell candidates apart
  __device__ static u32 key(u32 b, u32 inf) { return desc_key(b, inf); }
  __device__ static u32 prefix(u32 b, u32 inf) { return desc_key(b, inf); }
  __device__ static u64 pack(u32 b, u32 idx, u32 inf) { return pack_candidate(b, idx, inf); }
  __device__ static u32 index(u64 P) { return cand_index(P); }
  __device__ static u32 element(const u32 (&w4)[4], int e) { return (w4[e >> 1] >> ((e & 1) * 16)) & 0xffffu; }
  __device__ static void fill(u32 (&w4)[4], int e) { w4[e >> 1] |= 0xffffu << ((e & 1) * 16); }
};
struct Elem32 {
  static constexpr int kPerVec = 4;
  static constexpr int kBytes = 4;
  static constexpr int kKeyBits = 32;
  static constexpr int kIdxShift = 0;
  static constexpr int kLowDigit = 0;
  __device__ static u32 key(u32 b, u32) { return desc_key32(b); }
  __device__ static u32 prefix(u32 b, u32) { return desc_key32(b) >> 16; }
  __device__ static u64 pack(u32 b, u32 idx, u32) { return (static_cast<u64>(desc_key32(b)) << 32) | idx; }
  __device__ static u32 index(u64 P) { return static_cast<u32>(P); }
  __device__ static u32 element(const u32 (&w4)[4], int e) { return w4[e]; }
  __device__ static void fill(u32 (&w4)[4], int e) { w4[e] = 0xffffffffu; }
};

// ------------------------------------------------------------------------------ wave64 helpers

__device__ __forceinline__ u64 ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

__device__ __forceinline__ u32 mbcnt(u64 m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<u32>(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<u32>(m), 0u));
}

__device__ __forceinline__ u64 shfl_xor_u64(u64 x, int mask, int lane) {
  const int src = (lane ^ mask) << 2;
  const u32 lo = static_cast<u32>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(static_cast<u32>(x))));
  const u32 hi = static_cast<u32>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(static_cast<u32>(x >> 32))));
  return (static_cast<u64>(hi) << 32) | lo;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ u32 dpp(u32 x) {
  return static_cast<u32>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, ROW_MASK, 0xf, false));
}

// OR of x over the wave (DPP OR-scan; lane 63 holds the total), returned wave-uniform.
__device__ __forceinline__ u32 wave_or(u32 x) {
  x |= dpp<0x111, 0xf>(x);
  x |= dpp<0x112, 0xf>(x);
  x |= dpp<0x114, 0xf>(x);
  x |= dpp<0x118, 0xf>(x);
  x |= dpp<0x142, 0xa>(x);
  x |= dpp<0x143, 0xc>(x);
  return static_cast<u32>(__builtin_amdgcn_readlane(static_cast<int>(x), 63));
}

// One step of a wave minimum over u64 with DPP: lanes without a source lane (and rows the row
// mask leaves out) see ~0, the identity of the minimum.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ u64 dpp_min_u64(u64 x) {
  const u32 lo = static_cast<u32>(__builtin_amdgcn_update_dpp(-1, static_cast<int>(static_cast<u32>(x)), CTRL,
                                                               ROW_MASK, 0xf, false));
  const u32 hi = static_cast<u32>(__builtin_amdgcn_update_dpp(-1, static_cast<int>(static_cast<u32>(x >> 32)), CTRL,
                                                               ROW_MASK, 0xf, false));
  const u64 y = (static_cast<u64>(hi) << 32) | lo;
  return y < x ? y : x;
}

// Minimum of x over the wave (DPP min-scan; lane 63 holds it), returned wave-uniform.
__device__ __forceinline__ u64 wave_min_u64(u64 x) {
  x = dpp_min_u64<0x111, 0xf>(x);
  x = dpp_min_u64<0x112, 0xf>(x);
  x = dpp_min_u64<0x114, 0xf>(x);
  x = dpp_min_u64<0x118, 0xf>(x);
  x = dpp_min_u64<0x142, 0xa>(x);
  x = dpp_min_u64<0x143, 0xc>(x);
  const u32 lo = static_cast<u32>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<u32>(x)), 63));
  const u32 hi = static_cast<u32>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<u32>(x >> 32)), 63));
  return (static_cast<u64>(hi) << 32) | lo;
}

// Inclusive prefix sum across a wave64 with DPP: row_shr 1/2/4/8 inside each 16-lane row,
// then row_bcast:15 and row_bcast:31 carry the row totals upward.
__device__ __forceinline__ u32 wave_inclusive_scan(u32 x) {
  x += dpp<0x111, 0xf>(x);
  x += dpp<0x112, 0xf>(x);
  x += dpp<0x114, 0xf>(x);
  x += dpp<0x118, 0xf>(x);
  x += dpp<0x142, 0xa>(x);
  x += dpp<0x143, 0xc>(x);
  return x;
}


// ------------------------------------------------------------------------------ LDS layout

struct Smem {
  u32* hist;    // [256]
  u32* hist2;   // [256]
  int* scal;    // [32]
  u32* wcnt;    // [16] (cooperative: words 0-1 hold the call token)
  u64* area;    // [kArea] contiguous candidate list
  u64* sel;     // [kpad]
  int* rank;    // [max(kpad, kRankCap)]
  u32* stage;   // [NW][kStageWords] per-wave filter regions
};

__device__ __forceinline__ Smem carve_smem(unsigned char* smem, int kpad) {
  Smem s;
  s.hist = reinterpret_cast<u32*>(smem);
  s.hist2 = s.hist + 256;
  s.scal = reinterpret_cast<int*>(s.hist2 + 256);
  s.wcnt = reinterpret_cast<u32*>(s.scal + 32);
  s.area = reinterpret_cast<u64*>(s.wcnt + 16);
  s.sel = s.area + kArea;
  s.rank = reinterpret_cast<int*>(s.sel + kpad);
  s.stage = reinterpret_cast<u32*>(s.rank + (kpad > kRankCap ? kpad : kRankCap));
  return s;
}

// Wave 0: find the histogram bucket holding the need-th (1-based) entry.  Writes
// out[0] = bucket, out[1] = entries in earlier buckets, out[2] = entries in the bucket.
__device__ __forceinline__ void wave_find_bucket(const u32* hist, int need, int* out, int lane) {
  const u32 c0 = hist[lane * 4 + 0], c1 = hist[lane * 4 + 1];
  const u32 c2 = hist[lane * 4 + 2], c3 = hist[lane * 4 + 3];
  const u32 sum = c0 + c1 + c2 + c3;
  const u32 incl = wave_inclusive_scan(sum);
  const u32 excl = incl - sum;
  const u32 uneed = static_cast<u32>(need);
  if (excl < uneed && uneed <= incl) {
    u32 run = excl;
    int b = lane * 4;
    u32 cnt = c0;
    if (run + c0 < uneed) {
      run += c0;
      b += 1;
      cnt = c1;
      if (run + c1 < uneed) {
        run += c1;
        b += 1;
        cnt = c2;
        if (run + c2 < uneed) {
          run += c2;
          b += 1;
          cnt = c3;
        }
      }
    }
    out[0] = b;
    out[1] = static_cast<int>(run);
    out[2] = static_cast<int>(cnt);
  }
}

// Exact radix select over M unique packed values in LDS: returns the bound B such that
// exactly kk values are <= B (1 <= kk <= M).  8-bit digits over the key and index fields,
// MSB first, early exit as soon as a bucket is taken whole.  Indices are below n, so the index
// bytes above n - 1's highest byte are zero in every entry and take no pass.
template <int BLOCK, class E>
__device__ u64 block_select_bound(const u64* list, int M, int kk, u32* hist, int* scal, int64_t n) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int idx_bytes = n <= 0x100 ? 1 : (n <= 0x10000 ? 2 : (n <= 0x1000000 ? 3 : 4));
  u64 prefix = 0, pmask = 0;
  int need = kk;
  for (int shift = 56; shift >= E::kLowDigit; shift -= 8) {
    if (shift < E::kIdxShift + 32 && (shift - E::kIdxShift) / 8 >= idx_bytes) {
      pmask |= 0xffull << shift;  // a zero index byte in every entry: digit 0, no pass
      continue;
    }
    for (int i = tid; i < 256; i += BLOCK) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < M; i += BLOCK) {
      const u64 P = list[i];
      if ((P & pmask) == prefix) atomicAdd(&hist[(P >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (wid == 0) wave_find_bucket(hist, need, scal, lane);
    __syncthreads();
    const int b = scal[0];
    const int before = scal[1];
    const int cnt = scal[2];
    need -= before;
    prefix |= static_cast<u64>(b) << shift;
    pmask |= 0xffull << shift;
    if (need == cnt) break;
  }
  return prefix | ~pmask;
}

// Writes the pad (index -1, all-ones value bits: a NaN) at output slot o; indices-only calls
// have no value array.
template <class E>
__device__ __forceinline__ void write_pad(const TopkParams& p, int64_t o) {
  p.out_idx[o] = -1;
  if (p.out_vals) {
    if constexpr (E::kBytes == 2) {
      static_cast<uint16_t*>(p.out_vals)[o] = 0xffffu;
    } else {
      static_cast<u32*>(p.out_vals)[o] = 0xffffffffu;
    }
  }
}

// Raw fp32 bits of a candidate: decoded from its key, except for the keys of +-0 and NaN,
// which merge several bit patterns; those are read back from the input.
__device__ __forceinline__ u32 raw32_of(const TopkParams& p, int seg, u32 idx, u64 P) {
  const u32 key = static_cast<u32>(P >> 32);
  if (key == 0xffffffffu || key == 0x7fffffffu) {
    const int64_t s0 = (p.offsets ? static_cast<int64_t>(p.offsets[seg]) : static_cast<int64_t>(seg) * p.seg_len) + p.elem0;
    return reinterpret_cast<const u32*>(p.base)[s0 + idx];
  }
  return (key & 0x80000000u) ? key : (key ^ 0x7fffffffu);
}

// Writes rank r of the segment's output row.  An entry outside the segment (only a padding
// sentinel can be) is written as the pad.
template <class E>
__device__ __forceinline__ void write_rank(const TopkParams& p, int64_t n, int seg, int r, u64 P) {
  const u32 idx = E::index(P);
  const int64_t o = static_cast<int64_t>(seg) * p.k + r;
  if (r >= p.k) return;
  if (static_cast<int64_t>(idx) < n) {
    p.out_idx[o] = static_cast<int>(idx);
    if (p.out_vals) {
      if constexpr (E::kBytes == 2) {
        static_cast<uint16_t*>(p.out_vals)[o] = static_cast<uint16_t>(cand_raw(P));
      } else {
        static_cast<u32*>(p.out_vals)[o] = raw32_of(p, seg, idx, P);
      }
    }
  } else {
    write_pad<E>(p, o);
  }
}

// rank[i] = #{j : v[j] < v[i]} over the M entries of v, comparisons split over all threads.
template <int BLOCK>
__device__ void block_rank(const u64* v, int M, int* rank) {
  const int tid = threadIdx.x;
  for (int i = tid; i < M; i += BLOCK) rank[i] = 0;
  __syncthreads();
  const int slices = BLOCK / M > 0 ? BLOCK / M : 1;
  const int span = (M + slices - 1) / slices;
  for (int t = tid; t < M * slices; t += BLOCK) {
    const int i = t % M;
    const int q = t / M;
    const int j0 = q * span;
    const int j1 = j0 + span < M ? j0 + span : M;
    const u64 P = v[i];
    int c = 0;
    for (int j = j0; j < j1; ++j) c += v[j] < P ? 1 : 0;
    if (slices == 1) {
      rank[i] = c;
    } else if (c) {
      atomicAdd(&rank[i], c);
    }
  }
  __syncthreads();
}

// Ranks the M unique entries of `list` (LDS, 16-byte aligned, M <= rank capacity) and writes
// those of rank < kk to the segment's output row (also to sorted[rank] when sorted is not
// null); rank(x) = #{j : list[j] < x}.  A wave takes 128 candidates, two per lane, and a share
// of the entries, which it reads as wave-uniform 16-byte LDS broadcasts (two entries each);
// every lane counts the entries below each of its candidates with one 64-bit compare and one
// add per entry.  That spreads the M * M comparisons over the VALUs of all four SIMDs instead of
// issuing a ballot popcount per (candidate, 64 entries) on the CU's single scalar unit.  The
// entry range is split between the waves that share a candidate group, and the partial counts
// are summed in rank[] (LDS, M ints) before the writes.
template <int BLOCK, class E>
__device__ void lds_rank_write(const TopkParams& p, int64_t n, int seg, const u64* list, int M,
                               int kk, int* rank, u64* sorted) {
  typedef u64 u64x2_t __attribute__((ext_vector_type(2)));
  constexpr int NW = BLOCK / 64;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int G = (M + 127) >> 7;                 // candidate groups of 128 (two per lane)
  const int Q = G >= NW ? 1 : NW / G;           // waves sharing one group's entry range
  const int span = ((M + Q - 1) / Q + 7) & ~7;  // entries per share, a multiple of 8
  for (int i = threadIdx.x; i < M; i += BLOCK) rank[i] = 0;
  __syncthreads();
  TOPK_WTRACE(6);
  const u64x2_t* pairs = reinterpret_cast<const u64x2_t*>(list);
  for (int u = wid; u < G * Q; u += NW) {
    const int g = u % G;
    const int q = u / G;
    const int i0 = g * 128 + lane;
    const int i1 = i0 + 64;
    const u64 x0 = i0 < M ? list[i0] : 0ull;
    const u64 x1 = i1 < M ? list[i1] : 0ull;
    const int j0 = q * span;
    const int j1 = j0 + span < M ? j0 + span : M;
    u32 c0 = 0, c1 = 0;
    int j = j0;
    // 16 entries (eight reads in flight) per step, then one step of 8: the loop is bound by
    // LDS latency, not by the compares, when a SIMD holds only two waves.
    for (; j + 16 <= j1; j += 16) {
      u64x2_t a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = pairs[(j >> 1) + e];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        c0 += (a[e].x < x0 ? 1u : 0u) + (a[e].y < x0 ? 1u : 0u);
        c1 += (a[e].x < x1 ? 1u : 0u) + (a[e].y < x1 ? 1u : 0u);
      }
    }
    if (j + 8 <= j1) {
      u64x2_t a[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = pairs[(j >> 1) + e];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        c0 += (a[e].x < x0 ? 1u : 0u) + (a[e].y < x0 ? 1u : 0u);
        c1 += (a[e].x < x1 ? 1u : 0u) + (a[e].y < x1 ? 1u : 0u);
      }
      j += 8;
    }
    for (; j < j1; ++j) {
      const u64 v = list[j];
      c0 += v < x0 ? 1u : 0u;
      c1 += v < x1 ? 1u : 0u;
    }
    if (i0 < M && c0) atomicAdd(&rank[i0], static_cast<int>(c0));
    if (i1 < M && c1) atomicAdd(&rank[i1], static_cast<int>(c1));
  }
  TOPK_WTRACE(7);
  __syncthreads();
  for (int i = threadIdx.x; i < M; i += BLOCK) {
    const int r = rank[i];
    if (r < kk) {
      const u64 x = list[i];
      write_rank<E>(p, n, seg, r, x);
      if (sorted) sorted[r] = x;
    }
  }
}

// lds_rank_write for 16-bit elements in segments of at most 65,536 elements: the count runs
// on 32-bit words (key16 << 16 | index16, ordered as the packed candidates are, since
// indices are unique) staged in `keys` (LDS, 16-byte aligned, M + 3 words), so one 16-byte
// broadcast read brings four entries and each compare is a 32-bit one.
template <int BLOCK, class E>
__device__ void lds_rank_write16(const TopkParams& p, int64_t n, int seg, const u64* list, int M,
                                 int kk, int* rank, u32* keys, u64* sorted) {
  constexpr int NW = BLOCK / 64;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int G = (M + 127) >> 7;                  // candidate groups of 128 (two per lane)
  const int Q = G >= NW ? 1 : NW / G;            // waves sharing one group's entry range
  const int span = ((M + Q - 1) / Q + 15) & ~15;  // entries per share, a multiple of 16
  for (int i = threadIdx.x; i < M; i += BLOCK) {
    const u64 P = list[i];
    keys[i] = (static_cast<u32>(P >> 48) << 16) | (static_cast<u32>(P >> 16) & 0xffffu);
    rank[i] = 0;
  }
  __syncthreads();
  TOPK_WTRACE(6);
  const uint4* quads = reinterpret_cast<const uint4*>(keys);
  for (int u = wid; u < G * Q; u += NW) {
    const int g = u % G;
    const int q = u / G;
    const int i0 = g * 128 + lane;
    const int i1 = i0 + 64;
    const u32 x0 = i0 < M ? keys[i0] : 0u;
    const u32 x1 = i1 < M ? keys[i1] : 0u;
    const int j0 = q * span;
    const int j1 = j0 + span < M ? j0 + span : M;
    u32 c0 = 0, c1 = 0;
    int j = j0;
    // 32 entries (eight reads in flight) per step, then steps of 4, then single entries
    for (; j + 32 <= j1; j += 32) {
      uint4 a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = quads[(j >> 2) + e];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        c0 += (a[e].x < x0 ? 1u : 0u) + (a[e].y < x0 ? 1u : 0u) + (a[e].z < x0 ? 1u : 0u) + (a[e].w < x0 ? 1u : 0u);
        c1 += (a[e].x < x1 ? 1u : 0u) + (a[e].y < x1 ? 1u : 0u) + (a[e].z < x1 ? 1u : 0u) + (a[e].w < x1 ? 1u : 0u);
      }
    }
    for (; j + 4 <= j1; j += 4) {
      const uint4 a = quads[j >> 2];
      c0 += (a.x < x0 ? 1u : 0u) + (a.y < x0 ? 1u : 0u) + (a.z < x0 ? 1u : 0u) + (a.w < x0 ? 1u : 0u);
      c1 += (a.x < x1 ? 1u : 0u) + (a.y < x1 ? 1u : 0u) + (a.z < x1 ? 1u : 0u) + (a.w < x1 ? 1u : 0u);
    }
    for (; j < j1; ++j) {
      const u32 v = keys[j];
      c0 += v < x0 ? 1u : 0u;
      c1 += v < x1 ? 1u : 0u;
    }
    if (i0 < M && c0) atomicAdd(&rank[i0], static_cast<int>(c0));
    if (i1 < M && c1) atomicAdd(&rank[i1], static_cast<int>(c1));
  }
  TOPK_WTRACE(7);
  __syncthreads();
  for (int i = threadIdx.x; i < M; i += BLOCK) {
    const int r = rank[i];
    if (r < kk) {
      const u64 x = list[i];
      write_rank<E>(p, n, seg, r, x);
      if (sorted) sorted[r] = x;
    }
  }
}

// The value of lane (lane ^ M) for the masks a sorting network of 64 lanes uses.  Inside a
// 16-lane row DPP moves it with no LDS round trip: quad permutations for 1, 2 and 3, the row
// half-mirror and mirror for 7 and 15, a row rotation for 8 and two rotations and a select
// for 4 (row_ror:n gives lane i the value of lane (i - n) mod 16).  Across rows a swizzle
// (16, 31, inside each half-wave) or a bpermute (63).
template <int CTRL>
__device__ __forceinline__ u32 dpp_mov(u32 x) {
  return static_cast<u32>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, 0xf, 0xf, false));
}
template <int M>
__device__ __forceinline__ u32 xor_lane(u32 x, int lane) {
  if constexpr (M == 1) {
    return dpp_mov<0xB1>(x);  // quad_perm [1,0,3,2]
  } else if constexpr (M == 2) {
    return dpp_mov<0x4E>(x);  // quad_perm [2,3,0,1]
  } else if constexpr (M == 3) {
    return dpp_mov<0x1B>(x);  // quad_perm [3,2,1,0]
  } else if constexpr (M == 4) {
    const u32 down = dpp_mov<0x124>(x);  // lane i - 4
    const u32 up = dpp_mov<0x12C>(x);    // lane i + 4 (i - 12 mod 16)
    return (lane & 4) ? down : up;
  } else if constexpr (M == 7) {
    return dpp_mov<0x141>(x);  // row_half_mirror
  } else if constexpr (M == 8) {
    return dpp_mov<0x128>(x);  // row_ror:8
  } else if constexpr (M == 15) {
    return dpp_mov<0x140>(x);  // row_mirror
  } else if constexpr (M == 16 || M == 31) {
    return static_cast<u32>(__builtin_amdgcn_ds_swizzle(static_cast<int>(x), (M << 10) | 0x1F));
  } else {
    static_assert(M == 63, "lane masks of the 64-lane network");
    return static_cast<u32>(__builtin_amdgcn_ds_bpermute((lane ^ 63) << 2, static_cast<int>(x)));
  }
}

// One compare-exchange step of an ascending sorting network across the wave (one u64 per
// lane, all values distinct or equal pads): lane i pairs with lane i ^ M, and of each pair the
// lane whose bit HI is clear keeps the smaller value.
template <int M, int HI>
__device__ __forceinline__ u64 sort_step(u64 x, int lane) {
  const u32 ylo = xor_lane<M>(static_cast<u32>(x), lane);
  const u32 yhi = xor_lane<M>(static_cast<u32>(x >> 32), lane);
  const u64 y = (static_cast<u64>(yhi) << 32) | ylo;
  const bool take = (y < x) != ((lane & HI) != 0);
  return take ? y : x;
}

// Ascending bitonic sort of one u64 per lane across a wave64, in the form whose comparators
// all point one way: merging two sorted runs of K/2 starts with the mirror step (lane i
// against lane i ^ (K - 1)), then half-cleaners K/4 .. 1.  21 steps; 18 of them stay in DPP.
__device__ __forceinline__ u64 wave_sort64(u64 x, int lane) {
  x = sort_step<1, 1>(x, lane);
  x = sort_step<3, 2>(x, lane);
  x = sort_step<1, 1>(x, lane);
  x = sort_step<7, 4>(x, lane);
  x = sort_step<2, 2>(x, lane);
  x = sort_step<1, 1>(x, lane);
  x = sort_step<15, 8>(x, lane);
  x = sort_step<4, 4>(x, lane);
  x = sort_step<2, 2>(x, lane);
  x = sort_step<1, 1>(x, lane);
  x = sort_step<31, 16>(x, lane);
  x = sort_step<8, 8>(x, lane);
  x = sort_step<4, 4>(x, lane);
  x = sort_step<2, 2>(x, lane);
  x = sort_step<1, 1>(x, lane);
  x = sort_step<63, 32>(x, lane);
  x = sort_step<16, 16>(x, lane);
  x = sort_step<8, 8>(x, lane);
  x = sort_step<4, 4>(x, lane);
  x = sort_step<2, 2>(x, lane);
  x = sort_step<1, 1>(x, lane);
  return x;
}

// Ranks the M (<= BLOCK, at most 16 runs of 64) unique entries of `list` (LDS) and writes those
// of rank < kk to the segment's output row (also to sorted[rank] when sorted is not null).
// Wave w sorts entries [64w, 64w + 64) in registers (wave_sort64; entries past M padded with
// ~0, which no candidate equals) and writes the sorted run back in place.  The rank of an
// entry is then the number of entries below it in every run, its own included (where that is
// its position): a 7-step binary search per run, eight runs' searches interleaved so their
// LDS reads are in flight together.  About M * runs * 7 LDS reads in place of the M * M
// compares of counting against every entry.
template <int BLOCK, class E>
__device__ __forceinline__ void sort_rank_write(const TopkParams& p, int64_t n, int seg, u64* list, int M, int kk,
                                                u64* sorted) {
  constexpr int NW = BLOCK / 64;
  static_assert(NW <= 16, "at most 16 runs");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int R = (M + 63) >> 6;  // runs
  if (wid < R) {
    const u64 x = tid < M ? list[tid] : ~0ull;
    list[tid] = wave_sort64(x, lane);
  }
  __syncthreads();
  if (wid < R) {  // every slot of the R runs (the padding holds ~0)
    const u64 x = list[tid];
    if (x != ~0ull) {
      int r = 0;
      for (int b0 = 0; b0 < R; b0 += 8) {  // uniform
        const u64* run[8];
        int pos[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          run[i] = list + 64 * (b0 + i < R ? b0 + i : wid);  // past R: a real run, not counted
          pos[i] = 0;
        }
        // entries of each run below x: pos advances by s while entry pos + s - 1 is below x
#pragma unroll
        for (int s = 32; s > 0; s >>= 1) {
#pragma unroll
          for (int i = 0; i < 8; ++i) pos[i] += run[i][pos[i] + s - 1] < x ? s : 0;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          pos[i] += run[i][pos[i]] < x ? 1 : 0;  // pos <= 63 here; all 64 below gives 64
          r += b0 + i < R ? pos[i] : 0;
        }
      }
      if (r < kk) {
        write_rank<E>(p, n, seg, r, x);
        if (sorted) sorted[r] = x;
      }
    }
  }
}

// The same network on one u32 per lane: a step is one lane move and a min, a max and a select
// (the u64 form needs two moves, a 64-bit compare and two selects).
template <int M, int HI>
__device__ __forceinline__ u32 sort_step32(u32 x, int lane) {
  const u32 y = xor_lane<M>(x, lane);
  const u32 lo = x < y ? x : y;
  const u32 hi = x < y ? y : x;
  return (lane & HI) ? hi : lo;
}
__device__ __forceinline__ u32 wave_sort64_u32(u32 x, int lane) {
  x = sort_step32<1, 1>(x, lane);
  x = sort_step32<3, 2>(x, lane);
  x = sort_step32<1, 1>(x, lane);
  x = sort_step32<7, 4>(x, lane);
  x = sort_step32<2, 2>(x, lane);
  x = sort_step32<1, 1>(x, lane);
  x = sort_step32<15, 8>(x, lane);
  x = sort_step32<4, 4>(x, lane);
  x = sort_step32<2, 2>(x, lane);
  x = sort_step32<1, 1>(x, lane);
  x = sort_step32<31, 16>(x, lane);
  x = sort_step32<8, 8>(x, lane);
  x = sort_step32<4, 4>(x, lane);
  x = sort_step32<2, 2>(x, lane);
  x = sort_step32<1, 1>(x, lane);
  x = sort_step32<63, 32>(x, lane);
  x = sort_step32<16, 16>(x, lane);
  x = sort_step32<8, 8>(x, lane);
  x = sort_step32<4, 4>(x, lane);
  x = sort_step32<2, 2>(x, lane);
  x = sort_step32<1, 1>(x, lane);
  return x;
}

// sort_rank_write for 16-bit candidates of a segment shorter than 65,535 elements: every
// candidate is ordered by the u32 key16 << 16 | index16 (unique, and never the padding ~0), so
// the runs are sorted and searched as u32 in `runs` (free LDS of M + 64 words); each thread
// keeps its u64 candidate for the output.
template <int BLOCK, class E>
__device__ __forceinline__ void sort_rank_write16(const TopkParams& p, int64_t n, int seg, const u64* list, int M,
                                                  int kk, u64* sorted, u32* runs) {
  constexpr int NW = BLOCK / 64;
  static_assert(NW <= 16, "at most 16 runs");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int R = (M + 63) >> 6;  // runs
  const u64 P = tid < M ? list[tid] : ~0ull;
  const u32 x = tid < M ? ((static_cast<u32>(P >> 48) << 16) | (static_cast<u32>(P >> 16) & 0xffffu)) : ~0u;
  if (wid < R) runs[tid] = wave_sort64_u32(x, lane);
  __syncthreads();
  if (tid < M) {
    int r = 0;
    for (int b0 = 0; b0 < R; b0 += 8) {  // uniform
      const u32* run[8];
      int pos[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        run[i] = runs + 64 * (b0 + i < R ? b0 + i : wid);  // past R: a real run, not counted
        pos[i] = 0;
      }
#pragma unroll
      for (int s = 32; s > 0; s >>= 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) pos[i] += run[i][pos[i] + s - 1] < x ? s : 0;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pos[i] += run[i][pos[i]] < x ? 1 : 0;
        r += b0 + i < R ? pos[i] : 0;
      }
    }
    if (r < kk) {
      write_rank<E>(p, n, seg, r, P);
      if (sorted) sorted[r] = P;
    }
  }
}

// Ranks the M (<= 16 * S) unique candidates of `list` and writes those of rank < kk (also to
// sorted[rank] when sorted is not null).  One DPP row (16 lanes) per candidate: lane q of the
// row compares it with entries q, q + 16, ... (S of them, held in registers, loaded once), and
// a row prefix sum leaves its rank in the row's last lane, which writes the output entry.  The
// rows take the candidates in turn.  The S loads are unconditional (all inside the candidate
// area) and masked past M, so the slot count, not branches, bounds the work.
template <int BLOCK, int S, class E>
__device__ void row_rank_write(const TopkParams& p, int64_t n, int seg, const u64* list, int M, int kk,
                               u64* sorted) {
  static_assert(16 * S <= kArea, "the unconditional loads stay inside the candidate area");
  constexpr int ROWS = BLOCK / 16;
  const int row = threadIdx.x >> 4;
  const int q = threadIdx.x & 15;
  u64 ent[S];
#pragma unroll
  for (int t = 0; t < S; ++t) {
    const int i = q + 16 * t;
    const u64 e = list[i];
    ent[t] = i < M ? e : ~0ull;
  }
  TOPK_WTRACE(6);
  for (int c = row; c < M; c += ROWS) {  // uniform within each row
    const u64 x = list[c];
    u32 cnt = 0;
#pragma unroll
    for (int t = 0; t < S; ++t) cnt += ent[t] < x ? 1u : 0u;
    cnt += dpp<0x111, 0xf>(cnt);
    cnt += dpp<0x112, 0xf>(cnt);
    cnt += dpp<0x114, 0xf>(cnt);
    cnt += dpp<0x118, 0xf>(cnt);
    if (q == 15 && cnt < static_cast<u32>(kk)) {
      write_rank<E>(p, n, seg, static_cast<int>(cnt), x);
      if (sorted) sorted[cnt] = x;
    }
  }
  TOPK_WTRACE(7);
}

// Writes the top-k sampling draw of segment `seg` from its ranked entries sorted[0..kk)
// (wave 0), or the empty-row draw when kk is 0.  Only called when p.samples is set.
__device__ __forceinline__ void sample_segment(const TopkParams& p, const u64* sorted, int kk, int seg) {
  if (threadIdx.x >= 64) return;
  const bool bf16 = p.inf_bits == kInfBitsBF16;
  auto get = [&](int r) {
    const u64 P = sorted[r];
    return RankedEntry{bits16_to_float(cand_raw(P), bf16), static_cast<int32_t>(cand_index(P))};
  };
  sample_ranked_row(get, kk, p.k, p.inv_temperature, p.uniforms[seg], p.samples + seg,
                    p.probs ? p.probs + static_cast<int64_t>(seg) * p.k : nullptr);
}

// Select the kk best of the M packed candidates in `sm.area` (M >= kk) and write them, in
// order, to the segment's output row; ranks kk..k-1 get the pad (index -1, bits 0xFFFF).
// An unsorted call writes the same kk entries to slots 0..kk-1 in unspecified order when the
// list is too long for the rankers (shorter lists are ranked anyway: the ranking is the
// selection, and faster than a radix select).
// With top-k sampling on, the ranked entries are also kept in LDS (sm.sel, or sm.area when
// sm.sel holds the selection) and wave 0 then draws the segment's sample.
template <int BLOCK, class E>
__device__ __forceinline__ void finalize_segment(const TopkParams& p, const Smem& sm, int M, int kk, int64_t n,
                                 int seg) {
  const int tid = threadIdx.x;
  if (M < kk) kk = M;  // cannot happen (every candidate list holds >= kk entries); keeps it safe
  for (int r = kk + tid; r < p.k; r += BLOCK) {
    const int64_t o = static_cast<int64_t>(seg) * p.k + r;
    write_pad<E>(p, o);
  }
  const bool sampling = E::kBytes == 2 && p.samples != nullptr;  // 16-bit formats only
  constexpr int NW = BLOCK / 64;
  u64* sorted = sm.sel;
  // Small sets: one DPP row per candidate counts the smaller entries (row_rank_write).
  if (M <= 128) {
    if (M <= 64) {
      row_rank_write<BLOCK, 4, E>(p, n, seg, sm.area, M, kk, sampling ? sorted : nullptr);
    } else {
      row_rank_write<BLOCK, 8, E>(p, n, seg, sm.area, M, kk, sampling ? sorted : nullptr);
    }
  } else if (NW >= 8 && M <= 32 * NW && M <= kRankCap) {
    // Up to 32 entries per wave: rank the whole list (a radix select first, then ranking only
    // kk, was measured no faster: tied keys take the select through the index digits).  Longer
    // lists take the select: with 8 waves, ranking 512 entries in full (8 latency-bound LDS
    // passes per wave, two waves per SIMD) ran 66.7 -> 112.3 us on 6000 x 10000, k = 50.
    // Counting costs M * M compares, VALU-bound on the four SIMDs (about 2 us at M = 370);
    // sorted runs cost a fixed 21 DPP steps and 7 LDS levels.  Measured on 256 x 32000 fp16
    // rows of 256 distinct values: k = 256 (lists of about 370) 11.2 -> 9.4 us and k = 128
    // 9.5 -> 9.2 us with runs; with runs from 129 or 160 entries on, k = 64 lost 0.2-0.5 us.
    if (M >= kSortRankMin && E::kBytes == 2 && n < 0xffff) {
      sort_rank_write16<BLOCK, E>(p, n, seg, sm.area, M, kk, sampling ? sorted : nullptr, sm.stage);
    } else if (M >= kSortRankMin) {
      sort_rank_write<BLOCK, E>(p, n, seg, sm.area, M, kk, sampling ? sorted : nullptr);
    } else if (E::kBytes == 2 && n <= 0x10000) {
      lds_rank_write16<BLOCK, E>(p, n, seg, sm.area, M, kk, sm.rank, sm.stage, sampling ? sorted : nullptr);
    } else {
      lds_rank_write<BLOCK, E>(p, n, seg, sm.area, M, kk, sm.rank, sampling ? sorted : nullptr);
    }
  } else if (p.unsorted && !sampling) {
    // Unsorted output of a list too long for the rankers above: the kk best, found by radix
    // select, in the order they are found.  (Where the rankers apply they are faster than the
    // select: 256 x 32,000 fp16 rows of 256 distinct values, k = 256, 10.03 us unsorted by
    // select against 9.38 us ranked.)
    if (M > kk) {
      const u64 bound = block_select_bound<BLOCK, E>(sm.area, M, kk, sm.hist, sm.scal, n);
      if (tid == 0) sm.scal[3] = 0;
      __syncthreads();
      for (int i = tid; i < M; i += BLOCK) {
        const u64 P = sm.area[i];
        if (P <= bound) write_rank<E>(p, n, seg, atomicAdd(&sm.scal[3], 1), P);
      }
    } else {
      for (int i = tid; i < M; i += BLOCK) write_rank<E>(p, n, seg, i, sm.area[i]);
    }
  } else {
    const u64* sel = sm.area;
    if (M > kk) {
      const u64 bound = block_select_bound<BLOCK, E>(sm.area, M, kk, sm.hist, sm.scal, n);
      if (tid == 0) sm.scal[3] = 0;
      __syncthreads();
      for (int i = tid; i < M; i += BLOCK) {
        const u64 P = sm.area[i];
        if (P <= bound) {
          const int slot = atomicAdd(&sm.scal[3], 1);
          if (slot < p.kpad) sm.sel[slot] = P;
        }
      }
      __syncthreads();
      sel = sm.sel;
      sorted = sm.area;  // the candidates are no longer needed
    }
    // The kk selected entries: one thread per (entry, slice of the selection); ranking
    // them with lds_rank_write instead was measured slower on many short segments
    // (6000 x 10000, k = 50: 66.4 -> 68.0 us).
    block_rank<BLOCK>(sel, kk, sm.rank);
    for (int i = tid; i < kk; i += BLOCK) {
      write_rank<E>(p, n, seg, sm.rank[i], sel[i]);
      if (sampling) sorted[sm.rank[i]] = sel[i];
    }
  }
  if constexpr (E::kBytes == 2) {
    if (sampling) {
      __syncthreads();
      sample_segment(p, sorted, kk, seg);
    }
  }
}

// Epoch-tagged arrival counter: word = epoch << 16 | count.  A word carrying another epoch
// is stale (earlier call, or uninitialised workspace) and counts as zero.  The last
// arriver resets the count to zero, so a replay with the same epoch also works.
//
// Cross-workgroup publication protocol.  Every word one workgroup writes for another
// (list entries, list counts, this ticket) is an agent-scope atomic, which gfx950 lowers to
// device-coherent (sc1) vector memory accesses.  The writer waits for its stores to complete
// (s_waitcnt vmcnt(0)) before its arrival CAS, and the merger only issues its sc1 loads after
// its own CAS returned.  That is the agent-scope release/acquire pair restricted to sc1
// accesses, without the whole-L2 writeback (buffer_wbl2) and invalidate (buffer_inv) the
// generic fences add for plain stores and loads.
__device__ __forceinline__ bool arrive_last(u64* ticket, u64 epoch, int arrivals) {
  u64 old = __hip_atomic_load(ticket, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    const u64 cnt = ((old >> 16) == epoch) ? (old & 0xffffu) : 0u;
    const u64 next = cnt + 1u;
    const bool last = next >= static_cast<u64>(arrivals);
    const u64 word = (epoch << 16) | (last ? 0u : next);
    if (__hip_atomic_compare_exchange_strong(ticket, &old, word, __ATOMIC_RELAXED,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
      return last;
    }
  }
}

// Two-chunk segments.  Each workgroup swaps its mark (call epoch, chunk) into the segment's
// ticket; the one that gets the other chunk's mark back arrived second and merges, and it
// resets the ticket to zero.  A ticket left by any other call (or by the counter above, whose
// low 16 bits are zero after each call) never equals a mark of this one.
__device__ __forceinline__ u64 pair_mark(u64 epoch, int w) {
  return (epoch << 2) | static_cast<u64>(w + 1);
}
// Published entries carry a tag in bits 18..31 of their index field (two-chunk segments have
// indices below 2^18) with the top bit set, which no plain index has; the length word carries
// a 16-bit tag with the top bit set above the length.
template <class E>
constexpr u64 pair_tag_mask() { return 0x3fffull << (E::kIdxShift + 18); }
template <class E>
__device__ __forceinline__ u64 pair_entry_tag(u64 epoch) {
  return (0x2000ull | (epoch & 0x1fffu)) << (E::kIdxShift + 18);
}
__device__ __forceinline__ u32 pair_count_tag(u64 epoch) {
  return 0x8000u | static_cast<u32>(epoch & 0x7fffu);
}

// Orders a wave's LDS writes before its lanes read each other's entries (and the reads before
// the next overwrite): LDS requests of one wave are served in order, so this only has to keep
// the compiler from moving them across.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void wait_vector_memory() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ------------------------------------------------------------------------------ cooperative

// Per-segment block of the cooperative path (layout in topk_common.hpp).
struct GroupWs {
  u64* flag;    // tagged "histograms cleared"
  u64* gen;     // generation word: advanced once per call
  u64* arrive;  // [kGroupBarriers][W] arrival slots
  u64* counts;  // [2][W] epoch-tagged list lengths
  u32* hist;    // [kGroupCopies][256]
  u32* fine;    // [kFineCopies][kFineBins]
  u32* rhist;   // [6][256]
  u64* lists;   // [W][kCandArea]
};

__device__ __forceinline__ GroupWs group_ws(const TopkParams& p, int seg, int members) {
  const GroupLayout L = group_layout(members);
  unsigned char* b = p.groups + static_cast<size_t>(seg) * L.bytes;
  GroupWs g;
  g.flag = reinterpret_cast<u64*>(b + L.flag);
  g.gen = g.flag + 1;
  g.arrive = reinterpret_cast<u64*>(b + L.arrive);
  g.counts = reinterpret_cast<u64*>(b + L.counts);
  g.hist = reinterpret_cast<u32*>(b + L.hist);
  g.fine = reinterpret_cast<u32*>(b + L.fine);
  g.rhist = reinterpret_cast<u32*>(b + L.rhist);
  g.lists = reinterpret_cast<u64*>(b + L.lists);
  return g;
}

__device__ __forceinline__ u64 load_agent(const u64* a) {
  return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u32 load_agent(const u32* a) {
  return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(u64* a, u64 v) {
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(u32* a, u32 v) {
  __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Tagged words (tag44 << 20 | value20): a word carrying another tag is stale (an earlier call,
// or uninitialised workspace) and reads as "absent".
constexpr u64 kTagMask = (1ull << 44) - 1;
constexpr u32 kAbsent = 0xffffffffu;
constexpr u32 kGaveUp = 0xfffffffeu;  // group_collect: a bounded wait gave up
__device__ __forceinline__ u32 tagged_value(u64 word, u64 tag) {
  return (word >> 20) == tag ? static_cast<u32>(word & 0xfffffu) : kAbsent;
}

// Token of one cooperative call: the host's call epoch (unique per call made from the host)
// mixed with the segment block's generation word (advanced by every call, so unique per
// replay of a captured call, whose epoch is frozen).  Its low 44 bits (the tag of tagged
// words) are never zero, so a zeroed workspace holds no word of any call.
__device__ __forceinline__ u64 call_token(u64 epoch, u64 gen) {
  u64 t = epoch ^ (gen * 0x9E3779B97F4A7C15ull);
  if ((t & kTagMask) == 0) t |= 1u;
  return t;
}

// All `arrivals` workgroups of a segment meet here.  Each writes this call's token into its
// own arrival slot (no two workgroups touch one address), and threads 0..arrivals-1 each wait
// for one slot to hold `expect` (the token; anything else only under the test hook).  Every
// thread first waits for its own cross-workgroup writes (agent-scope atomics,
// device-coherent) to complete; after the barrier the workgroup's agent-scope loads see every
// other workgroup's writes.  Each wait is bounded by `limit` polls; returns false
// (workgroup-uniform) when one gave up.
__device__ __forceinline__ bool group_barrier(u64* slots, u64 token, u64 expect, int w, int arrivals,
                                              u32 limit) {
  wait_vector_memory();
  __syncthreads();
  const int tid = threadIdx.x;
  if (tid == 0) store_agent(slots + w, token);
  int late = 0;
  if (tid < arrivals) {
    late = 1;
    for (u32 spin = 0; spin < limit; ++spin) {
      if (load_agent(slots + tid) == expect) {
        late = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  return __syncthreads_or(late) == 0;
}

// Threshold histogram of the whole segment: every workgroup adds its LDS histogram to copy
// (w mod kGroupCopies) of the global one (nonzero bins only), the workgroups meet, and each
// loads the sum of the copies back into LDS (four copies per thread, partial sums staged in
// `scratch`, 1024 words of LDS).  Returns false when the meeting gave up.
template <int BLOCK>
__device__ bool group_histogram(u32* lds_hist, u32* ghist, u32* scratch, u64* slots, u64 token,
                                u64 expect, int w, int arrivals, u32 limit) {
  constexpr int Q = BLOCK / 256;  // threads per bin in the copy sum
  static_assert(Q >= 1 && kGroupCopies % Q == 0, "the copy sum splits the copies over Q threads per bin");
  const int tid = threadIdx.x;
  if (tid < 256) {
    const u32 c = lds_hist[tid];
    if (c) {
      __hip_atomic_fetch_add(ghist + (w % kGroupCopies) * 256 + tid, c, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (!group_barrier(slots, token, expect, w, arrivals, limit)) return false;
  const int bin = tid & 255;
  const int q = tid >> 8;
  u32 part = 0;
#pragma unroll
  for (int c = 0; c < kGroupCopies / Q; ++c) part += load_agent(ghist + (q + Q * c) * 256 + bin);
  scratch[q * 256 + bin] = part;
  __syncthreads();
  if (tid < 256) {
    u32 sum = 0;
#pragma unroll
    for (int i = 0; i < Q; ++i) sum += scratch[i * 256 + tid];
    lds_hist[tid] = sum;
  }
  __syncthreads();
  return true;
}

// Single-copy variant for the (rare) refinement digits.  Returns false when the meeting gave up.
template <int BLOCK>
__device__ bool group_histogram_single(u32* lds_hist, u32* ghist, u64* slots, u64 token, int w,
                                       int arrivals, u32 limit) {
  const int tid = threadIdx.x;
  if (tid < 256) {
    const u32 c = lds_hist[tid];
    if (c) __hip_atomic_fetch_add(ghist + tid, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!group_barrier(slots, token, token, w, arrivals, limit)) return false;
  if (tid < 256) lds_hist[tid] = load_agent(ghist + tid);
  __syncthreads();
  return true;
}

// Whole-segment candidate list from the workgroups' lists.  Each workgroup has stored its
// list and then, as its arrival, its tagged length: threads 0..arrivals-1 each wait for one
// length (no separate barrier), wave 0 prefix-sums them, and if no list overflowed and the
// total fits kGroupCap every entry is gathered into `area`.  Returns the total, kAbsent when
// the list cannot be formed, or kGaveUp when a wait for a length gave up (after `limit` polls;
// `want` is the tag of this call's lengths).  `cnt` and `pre` are 256-int LDS arrays.
template <int BLOCK>
__device__ u32 group_collect(const u64* counts, const u64* lists, u64 want, int arrivals, u64* area,
                             int* cnt, int* pre, int* scal, u32 limit) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  int late = 0;
  if (tid < 256) {
    u32 c = 0;
    if (tid < arrivals) {
      c = kAbsent;
      for (u32 spin = 0; spin < limit; ++spin) {
        c = tagged_value(load_agent(counts + tid), want);
        if (c != kAbsent) break;
        __builtin_amdgcn_s_sleep(1);
      }
      late = c == kAbsent ? 1 : 0;
      if (c > static_cast<u32>(kCandArea)) c = static_cast<u32>(kGroupCap) + 1u;  // overflow
    }
    cnt[tid] = static_cast<int>(c);
  }
  if (__syncthreads_or(late)) return kGaveUp;
  if (tid < 64) {
    const int c0 = cnt[4 * lane], c1 = cnt[4 * lane + 1], c2 = cnt[4 * lane + 2], c3 = cnt[4 * lane + 3];
    const u32 sum = static_cast<u32>(c0 + c1 + c2 + c3);
    const u32 incl = wave_inclusive_scan(sum);
    const u32 excl = incl - sum;
    pre[4 * lane] = static_cast<int>(excl);
    pre[4 * lane + 1] = static_cast<int>(excl + c0);
    pre[4 * lane + 2] = static_cast<int>(excl + c0 + c1);
    pre[4 * lane + 3] = static_cast<int>(excl + c0 + c1 + c2);
    if (lane == 63) scal[0] = static_cast<int>(incl);
  }
  __syncthreads();
  TOPK_TRACE(3);
  const u32 total = static_cast<u32>(scal[0]);
  if (total > static_cast<u32>(kGroupCap)) return kAbsent;
  // All of a thread's entries are located first and then loaded together, so their latencies
  // overlap.
  constexpr int kPer = (kGroupCap + BLOCK - 1) / BLOCK;
  const int rounds = static_cast<int>((total + BLOCK - 1) / BLOCK);  // workgroup-uniform
  size_t src[kPer];
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    src[r] = 0;
    if (r >= rounds) continue;
    const u32 i = static_cast<u32>(tid + r * BLOCK);
    int lo_t = 0, hi_t = arrivals;  // last t with pre[t] <= i
    while (hi_t - lo_t > 1) {
      const int mid = (lo_t + hi_t) >> 1;
      if (static_cast<u32>(pre[mid]) <= i) lo_t = mid; else hi_t = mid;
    }
    src[r] = static_cast<size_t>(lo_t) * kCandArea + (i - static_cast<u32>(pre[lo_t]));
  }
  u64 val[kPer];
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const u32 i = static_cast<u32>(tid + r * BLOCK);
    val[r] = i < total ? load_agent(lists + src[r]) : 0ull;
  }
#pragma unroll
  for (int r = 0; r < kPer; ++r) {
    const u32 i = static_cast<u32>(tid + r * BLOCK);
    if (i < total) area[i] = val[r];
  }
  __syncthreads();
  TOPK_TRACE(7);
  return total;
}

// Ranks the candidates list[c0, c1) against all M unique entries of `list` (LDS) and writes
// those of rank < kk to the output row: one wave per candidate, each lane comparing every
// 64th entry, the counts summed across the wave.
template <int BLOCK, class E>
__device__ void rank_range_write(const TopkParams& p, int64_t n, int seg, const u64* list, int M,
                                 int kk, int c0, int c1) {
  constexpr int NW = BLOCK / 64;
  const int lane = threadIdx.x & 63;
  const int wid = threadIdx.x >> 6;
  for (int i = c0 + wid; i < c1; i += NW) {
    const u64 P = list[i];
    u32 c = 0;
    for (int j = lane; j < M; j += 64) c += list[j] < P ? 1u : 0u;
    const u32 r = static_cast<u32>(__builtin_amdgcn_readlane(static_cast<int>(wave_inclusive_scan(c)), 63));
    if (lane == 0 && r < static_cast<u32>(kk)) write_rank<E>(p, n, seg, static_cast<int>(r), P);
  }
}

// A bounded cross-workgroup wait gave up: the workgroup fills its segment's row with the pad,
// records the timeout in the segment's status word (which the call reset before any of its
// workgroups could give up) and advances the segment block's generation word, if it has one,
// so the next call on this workspace uses a token no workgroup of this call has used.  The
// caller then returns without writing any other cross-workgroup word.
template <int BLOCK, class E>
__device__ void give_up_row(const TopkParams& p, int seg, u64* gen) {
  for (int r = threadIdx.x; r < p.k; r += BLOCK) write_pad<E>(p, static_cast<int64_t>(seg) * p.k + r);
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_or(p.status + seg, kStatusTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (gen) __hip_atomic_fetch_add(gen, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

__device__ __forceinline__ short2_t as_s2(u32 w) { return __builtin_bit_cast(short2_t, w); }
__device__ __forceinline__ u32 as_u32(short2_t w) { return __builtin_bit_cast(u32, w); }

// Packed int16 max / min of the 8 halves of a vector, as the two halves of one word.
__device__ __forceinline__ int vec_max4_i32(const uint4& x) {
  const int a = static_cast<int>(x.x) > static_cast<int>(x.y) ? static_cast<int>(x.x) : static_cast<int>(x.y);
  const int b = static_cast<int>(x.z) > static_cast<int>(x.w) ? static_cast<int>(x.z) : static_cast<int>(x.w);
  return a > b ? a : b;
}
__device__ __forceinline__ int vec_min4_i32(const uint4& x) {
  const int a = static_cast<int>(x.x) < static_cast<int>(x.y) ? static_cast<int>(x.x) : static_cast<int>(x.y);
  const int b = static_cast<int>(x.z) < static_cast<int>(x.w) ? static_cast<int>(x.z) : static_cast<int>(x.w);
  return a < b ? a : b;
}
// Larger half of a packed int16 pair.
__device__ __forceinline__ int vec_gmax(short2_t g) { return g.x > g.y ? g.x : g.y; }
__device__ __forceinline__ u32 vec_max2(const uint4& x) {
  return as_u32(__builtin_elementwise_max(__builtin_elementwise_max(as_s2(x.x), as_s2(x.y)),
                                          __builtin_elementwise_max(as_s2(x.z), as_s2(x.w))));
}
__device__ __forceinline__ u32 vec_min2(const uint4& x) {
  return as_u32(__builtin_elementwise_min(__builtin_elementwise_min(as_s2(x.x), as_s2(x.y)),
                                          __builtin_elementwise_min(as_s2(x.z), as_s2(x.w))));
}

// ------------------------------------------------------------------------------ the kernel

// At least 4 waves per SIMD (at most 128 VGPRs): one 1024-thread workgroup, or two 512-thread
// ones, per CU.  (Fewer, fatter waves -- 512 threads x 32 vectors -- measured slower.)
template <int BLOCK, int VPT, bool COOP, class E, bool SHORT = false>
__global__ void __launch_bounds__(BLOCK) __attribute__((amdgpu_waves_per_eu(4)))
segmented_topk_kernel(TopkParams p) {
  constexpr int NW = BLOCK / 64;
  constexpr int EV = E::kPerVec;  // elements per 16-byte vector
  constexpr int CH = BLOCK * VPT * EV;
  static_assert(CH <= 65536 * 2, "chunk positions must fit the refinement packing, and the "
                                 "indices of a two-chunk segment 18 bits");
  static_assert(NW <= 16, "at most 16 waves");
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const Smem sm = carve_smem(smem_raw, p.kpad);

  TOPK_TRACE(0);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  // Vector slot of thread tid's vector j: in block j of BLOCK vectors, slot tid rotated by
  // ROT * j.  A rotation by a multiple of 64 keeps each wave's 64 slots contiguous and leaves
  // block 0 as it is.  Without it, data whose period divides the BLOCK * EV-element block
  // stride (the reference bench's fill repeats every 2,048 elements) gives a thread the same
  // values in every vector, its best then summarises one vector, and the threshold from the
  // thread bests lets several times k candidates through (1,500 rows of 10,000 such elements:
  // 371 candidates a row against 53 on random data).  Only the one-workgroup-per-chunk kernels
  // of at most 8 vectors rotate: the 16-vector ones serve rows long enough that the threshold
  // comes from many distinct vectors anyway.
  constexpr int ROT = (!COOP && VPT <= 8) ? 64 : 0;
  auto vslot = [tid](int j) { return j * BLOCK + ((tid + ROT * j) & (BLOCK - 1)); };
  auto wslot = [wid](int j) { return j * BLOCK + ((wid * 64 + ROT * j) & (BLOCK - 1)); };
  const int W = p.chunks_per_seg;
  // Chunk-major grid: every segment's first chunk is dispatched before any second chunk, so
  // the workgroups of chunks a segment does not reach (they return at once) come last.
  const int w = W == 1 ? 0 : static_cast<int>(blockIdx.x) / p.seg_num;
  const int seg = W == 1 ? static_cast<int>(blockIdx.x) : static_cast<int>(blockIdx.x) - w * p.seg_num;
  const int k = p.k;
  const u32 inf = p.inf_bits;  // +inf bit pattern of the element format

  int64_t s0, s1;
  if (p.offsets) {
    s0 = p.offsets[seg];
    s1 = p.offsets[seg + 1];
    if (s1 < s0) s1 = s0;
  } else {
    s0 = static_cast<int64_t>(seg) * p.seg_len;
    s1 = s0 + p.seg_len;
  }
  s0 += p.elem0;
  s1 += p.elem0;
  const int64_t n = s1 - s0;
  const int64_t a0 = s0 & ~static_cast<int64_t>(EV - 1);
  const int64_t span_aligned = s1 - a0;
  const int64_t Ws64 = n > 0 ? (span_aligned + CH - 1) / CH : 0;

  if (n <= 0 || n > p.max_len || Ws64 > W) {
    // Empty segment, or one longer than the declared maximum (broken max_seg_len
    // precondition of the segmented entry point): the whole row is padding.
    if (w == 0) {
      for (int r = tid; r < k; r += BLOCK) {
        const int64_t o = static_cast<int64_t>(seg) * k + r;
        write_pad<E>(p, o);
      }
      if (tid == 0) store_agent(p.status + seg, kStatusOk);
      if constexpr (!COOP && E::kBytes == 2) {
        if (p.samples) sample_segment(p, nullptr, 0, seg);
      }
    }
    return;
  }
  const int Ws = static_cast<int>(Ws64);
  if (w >= Ws) return;
  // A segment of one chunk has no cross-workgroup wait: it completes.  (Multi-chunk segments
  // record their status where they merge, or, cooperatively, at the start.)
  if (!COOP && Ws == 1 && tid == 0) p.status[seg] = kStatusOk;

  const int kk = n < k ? static_cast<int>(n) : k;
  // A two-chunk segment merges through one published list (step 5).
  const bool pair = !COOP && BLOCK >= 512 && Ws == 2 && p.cap_list <= BLOCK;
  const int64_t cb = a0 + static_cast<int64_t>(w) * CH;
  const int64_t c0 = s0 > cb ? s0 : cb;
  const int64_t c1 = s1 < cb + CH ? s1 : cb + CH;
  const int nc = static_cast<int>(c1 - c0);
  const int kc = nc < k ? nc : k;
  const int lo = static_cast<int>(c0 - cb);  // valid chunk positions are [lo, hi)
  const int hi = static_cast<int>(c1 - cb);
  const u32 idx_base = static_cast<u32>(cb - s0);  // segment index = idx_base + position
  const int need = COOP ? kk : kc;  // rank the threshold must cover (segment or chunk)

  // Cooperative path: every workgroup reads the segment block's generation word and derives
  // the call token from it (thread 0, broadcast through LDS at the barrier below).  Workgroup 0
  // resets the segment's status, clears the segment's global histograms of this call before
  // loading its chunk, then raises the tagged "cleared" flag; once every workgroup has passed
  // the first barrier (and so has read the generation), it advances the generation for the
  // next call.
  const u64 epoch = p.epoch;
  u64 token = epoch;  // cooperative: this call's token (thread 0 until the broadcast)
  GroupWs g{};
  if constexpr (COOP) {
    g = group_ws(p, seg, p.chunks_per_seg);
    if (tid == 0) {
      token = call_token(epoch, load_agent(g.gen));
      reinterpret_cast<u64*>(sm.wcnt)[0] = token;
      if (w == 0) store_agent(p.status + seg, kStatusOk);
    }
    if (w == 0) {
      for (int i = tid; i < kGroupCopies * 256; i += BLOCK) store_agent(g.hist + i, 0u);
      for (int i = tid; i < kFineCopies * kFineBins; i += BLOCK) store_agent(g.fine + i, 0u);
      for (int i = tid; i < kRefineDigits * 256; i += BLOCK) store_agent(g.rhist + i, 0u);
      wait_vector_memory();
      __syncthreads();
      if (tid == 0) store_agent(g.flag, ((token & kTagMask) << 20) | 1u);
    }
  }

  // ---- 1. load the chunk: all nontemporal 16-byte loads issued before any is consumed.
  // Buffer loads from the chunk's base: vector j of thread tid is at byte
  // ((tid + ROT * j) mod BLOCK) * 16 (a VGPR) plus j * BLOCK * 16 (a scalar offset).  The
  // buffer ends at the first 8-block boundary at or past hi, so a vector wholly past the chunk
  // reads as zero without touching memory; the vector holding hi is read whole, as the
  // refinement re-read below also does.
  uint4 v[VPT];
  const unsigned char* cptr = reinterpret_cast<const unsigned char*>(p.base) + cb * E::kBytes;
  {
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(cptr), static_cast<short>(0), ((hi + EV - 1) & ~(EV - 1)) * E::kBytes,
        kBufferWord3);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const u32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (vslot(j) - j * BLOCK) * 16, j * BLOCK * 16, kCachePolicyNT);
      v[j] = make_uint4(t.x, t.y, t.z, t.w);
    }
  }
  // Two-chunk segment: its arrival ticket is taken now, while the loads are in flight.  The
  // workgroup that finds the other's mark arrived second and merges (step 5), gathering one
  // published entry per thread (cap_list <= BLOCK).  Both workgroups see the same parameters,
  // so both take this path or neither does.
  u64 pair_seen = 0;
  if (pair && tid == 0) {
    pair_seen = __hip_atomic_exchange(p.tickets + seg, pair_mark(epoch, w), __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
  }
  for (int i = tid; i < 256; i += BLOCK) sm.hist[i] = 0;
  if constexpr (COOP) {
    // the 32-key resolution histogram of the cooperative threshold, in the (still unused)
    // candidate area
    u32* fine = reinterpret_cast<u32*>(sm.area);
    for (int i = tid; i < kFineBins; i += BLOCK) fine[i] = 0;
  }
  __syncthreads();  // histograms cleared (the loads stay in flight)
  if constexpr (COOP) token = reinterpret_cast<const u64*>(sm.wcnt)[0];
  const u64 tag = token & kTagMask;
  TOPK_TRACE(12);
  // Positions outside [lo, hi) become the filler.  lo > 0 only in a segment's first chunk,
  // where it is below 8, so only vector 0 can start before lo; whether a vector index reaches
  // past hi is workgroup-uniform, so the per-lane test runs only for those vectors.
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    if ((j == 0 && lo > 0) || (j + 1) * BLOCK * EV > hi) {
      if (BLOCK <= 512 && j * BLOCK * EV >= hi) {
        // The whole block lies past the chunk (short rows of a batch planned for its longest,
        // the last blocks of a 10,000-element row on 256 x 8): the filler (all ones in every
        // format), with no per-lane test.  1024-thread kernels keep the one path: their
        // chunks rarely end a block early, and the extra branch cost 256 x 32,000 rows about
        // 0.1 us.
        v[j] = make_uint4(~0u, ~0u, ~0u, ~0u);
      } else {
        const int pos = vslot(j) * EV;
        if (pos < lo || pos + EV > hi) {
          u32 w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
          for (int e = 0; e < EV; ++e) {
            if (pos + e < lo || pos + e >= hi) E::fill(w4, e);
          }
          v[j] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
        }
      }
    }
  }

  // ---- 2. thread best (packed int16 max tree; for 32-bit elements an int32 one).  As
  // signed integers, the non-negative-sign elements order like their values, so the max is
  // the thread's best unless it has none: then its best is the min (the negative value
  // nearest zero), and only a wave holding such a lane builds the min tree.  Every VALU
  // instruction here costs all 4 waves of the SIMD.
  // Per-vector max as one int, kept for the filter's vector test: reducing it here, while
  // later waves' data is still in flight, leaves the filter one compare per vector.
  int gv[VPT];
  int m1, m2;
  if constexpr (E::kBytes == 2) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) gv[j] = vec_gmax(as_s2(vec_max2(v[j])));
    int mx = gv[0];
#pragma unroll
    for (int j = 1; j < VPT; ++j) mx = mx > gv[j] ? mx : gv[j];
    m1 = mx;  // int16 max: the best non-negative-sign half
    m2 = 32767;
    if (ballot(m1 < 0)) {
      short2_t mn = as_s2(vec_min2(v[0]));
#pragma unroll
      for (int j = 1; j < VPT; ++j) mn = __builtin_elementwise_min(mn, as_s2(vec_min2(v[j])));
      m2 = mn.x < mn.y ? mn.x : mn.y;
    }
  } else {
#pragma unroll
    for (int j = 0; j < VPT; ++j) gv[j] = vec_max4_i32(v[j]);
    int mx = gv[0];
#pragma unroll
    for (int j = 1; j < VPT; ++j) mx = mx > gv[j] ? mx : gv[j];
    m1 = mx;
    m2 = 0x7fffffff;
    if (ballot(m1 < 0)) {
      int mn = vec_min4_i32(v[0]);
#pragma unroll
      for (int j = 1; j < VPT; ++j) {
        const int t = vec_min4_i32(v[j]);
        mn = mn < t ? mn : t;
      }
      m2 = mn;
    }
  }
  const u32 best_bits = static_cast<u32>(m1 >= 0 ? m1 : m2) & (E::kBytes == 2 ? 0xffffu : 0xffffffffu);
  const u32 best_key = E::prefix(best_bits, inf);
  TOPK_TRACE(1);
  TOPK_WTRACE(1);

  // ---- k = 1 (16-bit single-chunk rows, no sampling): the chunk's best element directly.  T
  // is the smallest thread best key, a workgroup minimum (a thread best is a real element, so
  // the best element has key <= T).  For a positive T, the elements at or below it are found
  // as step 4 finds them (a vector can hold one only if its int16 max reaches raw(T), then an
  // exact test per element), and the smallest (key, position) of them is a second workgroup
  // minimum.  No list and no ranking.  A non-positive T (rows of no positive value) takes
  // the general path.
  if constexpr (!COOP && E::kBytes == 2) {
    if (k == 1 && Ws == 1 && !p.samples) {  // workgroup-uniform
      u64* wmin = sm.area;  // [NW] per-wave minima
      const u64 wt = wave_min_u64(best_key);
      if (lane == 0) wmin[wid] = wt;
      __syncthreads();
      u32 Ta = 0xffffffffu;
#pragma unroll
      for (int q = 0; q < NW; ++q) Ta = static_cast<u32>(wmin[q]) < Ta ? static_cast<u32>(wmin[q]) : Ta;
      if (Ta < 0x7fffu) {  // workgroup-uniform
        const u32 t_lo = Ta ^ 0x7fffu;  // raw bits of T: candidates are b in [t_lo, inf]
        const u32 span = inf - t_lo;
        u64 mine = ~0ull;  // this thread's smallest (key << 32 | position) at or below T
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
          if (gv[j] >= static_cast<int>(t_lo)) {
            const u32 w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
            for (int e = 0; e < EV; ++e) {
              const u32 b = E::element(w4, e);
              if (b - t_lo <= span) {  // t_lo <= b <= inf, as unsigned
                const u64 P = (static_cast<u64>(b ^ 0x7fffu) << 32) | static_cast<u32>(vslot(j) * EV + e);
                mine = P < mine ? P : mine;
              }
            }
          }
        }
        const u64 wbest = wave_min_u64(mine);
        __syncthreads();  // every wave has read the thread-best minima
        if (lane == 0) wmin[wid] = wbest;
        __syncthreads();
        if (tid == 0) {
          u64 P = wmin[0];
#pragma unroll
          for (int q = 1; q < NW; ++q) P = wmin[q] < P ? wmin[q] : P;
          const u32 raw = static_cast<u32>(P >> 32) ^ 0x7fffu;
          p.out_idx[seg] = static_cast<int>(idx_base + static_cast<u32>(P));
          if (p.out_vals) static_cast<uint16_t*>(p.out_vals)[seg] = static_cast<uint16_t>(raw);
        }
        return;
      }
      __syncthreads();  // the general path reuses the candidate area
    }
  }

  // ---- 3. threshold T.  A single workgroup: the kc-th smallest thread best, exactly, by two
  // LDS histogram passes (high byte, then low byte inside the boundary bucket).  A cooperative
  // segment: the thread bests' high-byte histogram and a 32-key resolution one (key >> 5) are
  // summed over the segment's workgroups in one meeting; T is the last key of the fine bin
  // holding the kk-th best, so at least kk real elements are at or below it, and at most that
  // bin's other keys' worth of extra elements pass.
  //   A short chunk (every position in each thread's first vector, at most 4 * EV * kc of
  // them) ranks its elements instead of its thread bests: then few threads hold a real best,
  // and a thread-best threshold would let most of the chunk through.  At most EV LDS atomics
  // per thread, and T is the chunk's exact kc-th key prefix.  Compiled only into the SHORT
  // instantiations, which the launch picks when a chunk can be short (segmented input, or
  // rows this short): elsewhere the unused branch measurably slows the threshold step.
  constexpr bool kElemMode = !COOP && SHORT;
  const bool elem_mode = kElemMode && hi <= BLOCK * EV && nc <= 4 * EV * kc;  // workgroup-uniform
  u32 ekeys[EV];  // key prefixes of this thread's first vector (elem_mode), 0x10000 if outside
  if (__builtin_expect(elem_mode, 0)) {
    const u32 w4[4] = {v[0].x, v[0].y, v[0].z, v[0].w};
#pragma unroll
    for (int e = 0; e < EV; ++e) {
      const int pos = tid * EV + e;
      ekeys[e] = (pos >= lo && pos < hi) ? E::prefix(E::element(w4, e), inf) : 0x10000u;
      if (ekeys[e] < 0x10000u) atomicAdd(&sm.hist[ekeys[e] >> 8], 1u);
    }
  } else {
    atomicAdd(&sm.hist[best_key >> 8], 1u);
  }
  if (tid < 256) sm.hist2[tid] = 0;
  if (tid == 0) sm.scal[4] = 0;  // candidate list counter
  u32 T;
  if constexpr (COOP) {
    u32* fine = reinterpret_cast<u32*>(sm.area);
    atomicAdd(&fine[best_key >> 5], 1u);
    __syncthreads();
    int late = 0;
    if (tid == 0) {  // the global histograms are cleared
      const u32 want = (p.force_timeout & kForceFlagWait) ? 2u : 1u;
      late = 1;
      for (u32 spin = 0; spin < p.spin_limit; ++spin) {
        if (tagged_value(load_agent(g.flag), tag) == want) {
          late = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    if (__syncthreads_or(late)) {
      give_up_row<BLOCK, E>(p, seg, g.gen);
      return;
    }
    // this workgroup's nonzero fine bins into its copy; the coarse ones go in group_histogram
    for (int i = tid; i < kFineBins; i += BLOCK) {
      const u32 c = fine[i];
      if (c) {
        __hip_atomic_fetch_add(g.fine + (w % kFineCopies) * kFineBins + i, c, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    const u64 expect = (p.force_timeout & kForceBarrier) ? (token ^ 1u) : token;
    if (!group_histogram<BLOCK>(sm.hist, g.hist, sm.stage, g.arrive, token, expect, w, Ws, p.spin_limit)) {
      give_up_row<BLOCK, E>(p, seg, g.gen);
      return;
    }
    // Every workgroup has read the generation word: advance it for the next call.
    if (w == 0 && tid == 0) __hip_atomic_fetch_add(g.gen, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    TOPK_TRACE(8);
    if (wid == 0) wave_find_bucket(sm.hist, need, sm.scal + 8, lane);
    __syncthreads();
    TOPK_TRACE(2);
    const u32 b1 = static_cast<u32>(sm.scal[8]);
    // the 8 fine bins of bucket b1, summed over the copies (thread t: bin t & 7, copy t >> 3)
    if (tid < 8 * kFineCopies) {
      sm.stage[tid] = load_agent(g.fine + (tid >> 3) * kFineBins + b1 * 8 + (tid & 7));
    }
    __syncthreads();
    if (wid == 0) {
      u32 c = 0;
      if (lane < 8) {
#pragma unroll
        for (int q = 0; q < kFineCopies; ++q) c += sm.stage[q * 8 + lane];
      }
      const u32 incl = wave_inclusive_scan(c);
      const u32 rest = static_cast<u32>(need - sm.scal[9]);  // rank inside bucket b1
      const u64 m = ballot(lane < 8 && incl >= rest);
      if (lane == static_cast<int>(__builtin_ctzll(m))) sm.scal[12] = lane;
    }
    __syncthreads();
    T = (((b1 << 3) | static_cast<u32>(sm.scal[12])) << 5) | 31u;
    TOPK_TRACE(9);
  } else {
    __syncthreads();
    if (wid == 0) wave_find_bucket(sm.hist, need, sm.scal + 8, lane);
    __syncthreads();
    TOPK_TRACE(2);
    const u32 b1 = static_cast<u32>(sm.scal[8]);
    if (__builtin_expect(elem_mode, 0)) {
#pragma unroll
      for (int e = 0; e < EV; ++e) {
        if ((ekeys[e] >> 8) == b1) atomicAdd(&sm.hist2[ekeys[e] & 0xffu], 1u);
      }
    } else if ((best_key >> 8) == b1) {
      atomicAdd(&sm.hist2[best_key & 0xffu], 1u);
    }
    __syncthreads();
    if (wid == 0) wave_find_bucket(sm.hist2, need - sm.scal[9], sm.scal + 12, lane);
    __syncthreads();
    T = (b1 << 8) | static_cast<u32>(sm.scal[12]);
  }
  TOPK_TRACE(4);
  TOPK_WTRACE(0);

  // ---- 4. filter {key prefix <= T} into the contiguous LDS candidate list, packed as
  // (key16 << 48 | index32 << 16 | raw16), or (key32 << 32 | index32) for 32-bit elements.
  // Instruction counts matter more than latency here:
  // the 16 waves of a CU share its scalar unit and LDS, and each SIMD issues for 4 waves.
  const bool all_mode = T == 0xffffu;  // no usable threshold: fewer than kc bests, or NaNs
  // Each thread best with key <= T is an element with key <= T: when more of them exist than
  // list entries (ties, all-equal rows) the list overflows for certain, and the refinement
  // below takes over without filtering.  (Cooperative counts cover the whole segment.)
  const int npass = sm.scal[9] + sm.scal[13] + sm.scal[14];
  const bool sure_overflow = !COOP && !all_mode && npass > kArea;
  const bool filter = !all_mode && !sure_overflow;
  if (filter && T < 0x7fffu) {
    // T is a positive value: candidates are the b in [raw(T), inf] (positive, non-NaN).
    // A vector can hold one only if the int16 max of its halves is >= raw(T).  Each wave
    // copies its lanes' vectors that pass this test into an LDS staging list (one 16-byte
    // write per such vector), then tests the staged vectors one per lane: one packed
    // subtract d = b - raw(T) per word and two unsigned compares give the exact hits
    // (d <= inf - raw(T) holds exactly for raw(T) <= b <= inf).  A wave prefix sum
    // gives every hit its offset, and one LDS atomic per 64 staged vectors reserves the
    // wave's slots in the list.  For 32-bit elements the bound is raw(T) << 16 (the smallest
    // positive pattern whose key prefix is T) and the test one unsigned compare per word.
    const u32 t_lo = E::kBytes == 2 ? (T ^ 0x7fffu) : ((T ^ 0x7fffu) << 16);
    const ushort2_t tt = {static_cast<unsigned short>(t_lo), static_cast<unsigned short>(t_lo)};
    const u32 span = (E::kBytes == 2 ? inf : 0x7f800000u) - t_lo;
    const u32 span_hi = (span << 16) | 0xffffu;
    uint4* st_vec = reinterpret_cast<uint4*>(sm.stage + wid * kStageWords);
    u32* st_pos = sm.stage + wid * kStageWords + 256;
    TOPK_WTRACE(2);
    u32 nst = 0;  // staged vectors (wave-uniform)
    // Tests the nst staged vectors one per lane and appends their hits to the list.
    auto flush = [&]() {
      wave_lds_sync();
      u32 w4[4] = {0u, 0u, 0u, 0u};
      u32 hm = 0;  // hits among the elements of this lane's staged vector
      u32 p0 = 0;
      if (static_cast<u32>(lane) < nst) {
        const uint4 x = st_vec[lane];
        w4[0] = x.x; w4[1] = x.y; w4[2] = x.z; w4[3] = x.w;
        p0 = idx_base + st_pos[lane];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if constexpr (E::kBytes == 2) {
            const u32 d = __builtin_bit_cast(u32, __builtin_bit_cast(ushort2_t, w4[q]) - tt);
            hm |= static_cast<u32>(static_cast<unsigned short>(d) <= span) << (2 * q);
            hm |= static_cast<u32>(d <= span_hi) << (2 * q + 1);
          } else {
            hm |= static_cast<u32>(w4[q] - t_lo <= span) << q;
          }
        }
      }
      // List offsets: with at most one hit per lane (the usual case) a lane's offset is its
      // rank among the hit lanes; otherwise a wave prefix sum of the hit counts.
      const u64 hit_lanes = ballot(hm != 0u);
      if (hit_lanes) {
        u32 excl, total;
        if (ballot((hm & (hm - 1u)) != 0u) == 0) {
          excl = mbcnt(hit_lanes);
          total = static_cast<u32>(__popcll(hit_lanes));
        } else {
          const u32 cnt = static_cast<u32>(__builtin_popcount(hm));
          const u32 incl = wave_inclusive_scan(cnt);
          total = static_cast<u32>(__builtin_amdgcn_readlane(static_cast<int>(incl), 63));
          excl = incl - cnt;
        }
        u32 base = 0;
        if (lane == 0) base = atomicAdd(reinterpret_cast<u32*>(&sm.scal[4]), total);
        u32 o = __builtin_amdgcn_readfirstlane(base) + excl;
        while (hm) {
          const u32 e = static_cast<u32>(__builtin_ctz(hm));
          hm &= hm - 1u;
          const u32 pi = p0 + e;
          // the hit element, read back from the staged vector (cheaper than selecting it
          // from the registers by a lane-varying index)
          if constexpr (E::kBytes == 2) {
            const u32 b = reinterpret_cast<const uint16_t*>(st_vec + lane)[e];
            if (o < static_cast<u32>(kArea))
              sm.area[o] = (static_cast<u64>(((b ^ 0x7fffu) << 16) | (pi >> 16)) << 32) | ((pi << 16) | b);
          } else {
            const u32 b = reinterpret_cast<const u32*>(st_vec + lane)[e];
            if (o < static_cast<u32>(kArea)) sm.area[o] = (static_cast<u64>(b ^ 0x7fffffffu) << 32) | pi;
          }
          ++o;
        }
      }
      wave_lds_sync();
      nst = 0;
    };
    // Stage the passing vectors: one compare and ballot per vector gives the wave's passing
    // lanes, and a wave-uniform branch skips the vectors no lane passes.
    auto stage_vector = [&](int j) {  // inlined into unrolled loops: j is a constant
      const bool mine = gv[j] >= static_cast<int>(t_lo);
      const u64 m = ballot(mine);
      if (m) {
        const u32 c = static_cast<u32>(__popcll(m));
        if (nst + c > 64u) flush();
        if (mine) {
          const u32 slot = nst + mbcnt(m);
          st_vec[slot] = v[j];
          st_pos[slot] = static_cast<u32>(vslot(j) * EV);
        }
        nst += c;
      }
    };
#pragma unroll
    for (int j = 0; j < VPT; ++j) stage_vector(j);
    TOPK_WTRACE(3);
    if (nst) flush();
    TOPK_WTRACE(4);
  } else if (filter) {
    // T is +-0 or negative: candidates are every non-NaN positive and the b with
    // uint16(b) <= raw(T) (raw of the zero class taken as 0x8000); for 32-bit elements, the
    // b whose key prefix is <= T.  Each wave collects its hits
    // in a private LDS region (ballot/mbcnt slots), then reserves its share of the list with
    // one LDS atomic and copies the region there.
    constexpr int RC = kStageWords / 2;  // region capacity (u64 entries) per wave
    u64* region = reinterpret_cast<u64*>(sm.stage + wid * kStageWords);
    u32 wcount = 0;  // wave-uniform
    const u32 traw = T == 0x7fffu ? 0x8000u : T;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      // the wave's positions of vector j: skip the whole vector (wave-uniform) when none
      // is in [lo, hi), as in every vector of a short segment past its end
      const int wpos = wslot(j) * EV;
      if (wpos >= hi || wpos + 64 * EV <= lo) continue;
      const u32 w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int e = 0; e < EV; ++e) {
        const u32 b = E::element(w4, e);
        bool h;
        if constexpr (E::kBytes == 2) {
          h = b <= traw && (b & 0x7fffu) <= inf;
        } else {
          h = E::prefix(b, inf) <= T;
        }
        const u64 m = ballot(h);
        if (m) {
          if (h) {
            const u32 slot = wcount + mbcnt(m);
            if (slot < static_cast<u32>(RC))
              region[slot] = E::pack(b, idx_base + static_cast<u32>(vslot(j) * EV + e), inf);
          }
          wcount += static_cast<u32>(__popcll(m));
        }
      }
    }
    // A region that overflowed forces the exact refinement by pushing the count past kArea.
    const u32 amount = wcount > static_cast<u32>(RC) ? static_cast<u32>(kArea) + 1u : wcount;
    if (amount) {
      wave_lds_sync();
      u32 base = 0;
      if (lane == 0) base = atomicAdd(reinterpret_cast<u32*>(&sm.scal[4]), amount);
      base = __builtin_amdgcn_readfirstlane(base);
      if (wcount <= static_cast<u32>(RC)) {
        for (u32 i = lane; i < wcount; i += 64) {
          if (base + i < static_cast<u32>(kArea)) sm.area[base + i] = region[i];
        }
      }
    }
  }
  TOPK_TRACE(5);
  if (pair && tid == 0) {
    sm.scal[5] = pair_seen == pair_mark(epoch, 1 - w) ? 1 : 0;
    sm.scal[6] = 0;  // stale-word reports of the merger's poll
  }
  __syncthreads();
  TOPK_WTRACE(5);

  int C = all_mode ? 0 : (sure_overflow ? kArea + 1 : sm.scal[4]);
  const bool overflow = C > kArea;
  // Re-reads the chunk from memory and calls fn(raw bits, chunk position) for every element
  // in [lo, hi): the refinement passes do not keep the fast path's registers live.
  auto for_each_element = [&](auto&& fn) {
#pragma unroll 1
    for (int j = 0; j < VPT; ++j) {
      const int pos0 = vslot(j) * EV;
      if (pos0 < hi && pos0 + EV > lo) {
        const uint4 x = *reinterpret_cast<const uint4*>(cptr + static_cast<u32>(pos0) * E::kBytes);
        const u32 w4[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int e = 0; e < EV; ++e) {
          const int pos = pos0 + e;
          if (pos >= lo && pos < hi) fn(E::element(w4, e), pos);
        }
      }
    }
  };

  if constexpr (COOP) {
    // ---- 4c. cooperative segment: one candidate list for the whole segment.  Every
    // workgroup stores its list in its own slot with an epoch-tagged length (an overflowing or
    // threshold-less chunk stores an oversized length instead), the workgroups meet, and every
    // workgroup gathers the whole list into LDS.
    int* cnt = reinterpret_cast<int*>(sm.hist);   // [256] list lengths of the workgroups
    int* pre = reinterpret_cast<int*>(sm.hist2);  // [256] their exclusive prefix sums
    const u32 contrib = (all_mode || overflow) ? static_cast<u32>(kCandArea) + 1u : static_cast<u32>(C);
    u64* mylist = g.lists + static_cast<size_t>(w) * kCandArea;
    if (contrib <= static_cast<u32>(kCandArea)) {
      for (u32 i = tid; i < contrib; i += BLOCK) store_agent(mylist + i, sm.area[i]);
    }
    wait_vector_memory();  // the list is complete before its length announces it
    __syncthreads();
    if (tid == 0) store_agent(g.counts + w, (tag << 20) | contrib);
    TOPK_TRACE(10);
    const u64 want = (p.force_timeout & kForceCollect) ? (tag ^ 1u) : tag;
    u32 total = group_collect<BLOCK>(g.counts, g.lists, want, Ws, sm.area, cnt, pre, sm.scal + 20, p.spin_limit);
    if (total == kGaveUp) {
      give_up_row<BLOCK, E>(p, seg, g.gen);
      return;
    }
    if (total == kAbsent) {
      // ---- 4d. the list would not fit: exact radix refinement over the whole segment of
      // Q = key << 32 | index32 among the elements with key prefix <= T, one global histogram
      // per 8-bit digit, until at most kCandArea elements are <= the bound (so that any one
      // workgroup's share fits its own list).
      u64 prefix = 0, pmask = 0;
      int rneed = kk;
      int pass = 0;
      constexpr u64 kQMask = E::kKeyBits == 32 ? ~0ull : ((1ull << (32 + E::kKeyBits)) - 1);
      static_assert(E::kKeyBits / 8 + 4 <= kRefineDigits, "one histogram per digit of Q");
      for (int shift = E::kKeyBits + 24; shift >= 0; shift -= 8, ++pass) {
        for (int i = tid; i < 256; i += BLOCK) sm.hist[i] = 0;
        __syncthreads();
        for_each_element([&](u32 b, int pos) {
          const u64 Q = (static_cast<u64>(E::key(b, inf)) << 32) | (idx_base + static_cast<u32>(pos));
          if (E::prefix(b, inf) <= T && (Q & pmask) == prefix) atomicAdd(&sm.hist[(Q >> shift) & 255u], 1u);
        });
        __syncthreads();
        if (!group_histogram_single<BLOCK>(sm.hist, g.rhist + pass * 256, g.arrive + (3 + pass) * W, token, w,
                                           Ws, p.spin_limit)) {
          give_up_row<BLOCK, E>(p, seg, g.gen);
          return;
        }
        if (wid == 0) wave_find_bucket(sm.hist, rneed, sm.scal, lane);
        __syncthreads();
        const int b = sm.scal[0];
        const int before = sm.scal[1];
        const int cnt_b = sm.scal[2];
        __syncthreads();
        rneed -= before;
        prefix |= static_cast<u64>(b) << shift;
        pmask |= 0xffull << shift;
        if ((kk - rneed) + cnt_b <= kCandArea) break;  // fits every workgroup's own list
      }
      const u64 bound = prefix | (~pmask & kQMask);
      if (tid == 0) sm.scal[4] = 0;
      __syncthreads();
      for_each_element([&](u32 b, int pos) {
        const u32 idx = idx_base + static_cast<u32>(pos);
        const u64 Q = (static_cast<u64>(E::key(b, inf)) << 32) | idx;
        if (E::prefix(b, inf) <= T && Q <= bound) {
          const int slot = atomicAdd(&sm.scal[4], 1);
          if (slot < kArea) sm.area[slot] = E::pack(b, idx, inf);
        }
      });
      __syncthreads();
      const u32 c2 = static_cast<u32>(sm.scal[4] < kArea ? sm.scal[4] : kArea);
      for (u32 i = tid; i < c2; i += BLOCK) store_agent(mylist + i, sm.area[i]);
      wait_vector_memory();
      __syncthreads();
      if (tid == 0) store_agent(g.counts + W + w, (tag << 20) | c2);
      total = group_collect<BLOCK>(g.counts + W, g.lists, tag, Ws, sm.area, cnt, pre, sm.scal + 20, p.spin_limit);
      if (total == kGaveUp) {
        give_up_row<BLOCK, E>(p, seg, g.gen);
        return;
      }
      if (total == kAbsent) total = 0;  // cannot happen: at most kCandArea elements are <= bound
    }
    // Every workgroup ranks its share of the list; workgroup 0 writes the pads.
    if (w == 0) {
      for (int r = kk + tid; r < k; r += BLOCK) {
        const int64_t o = static_cast<int64_t>(seg) * k + r;
        write_pad<E>(p, o);
      }
    }
    const int per = (static_cast<int>(total) + Ws - 1) / Ws;
    const int c0 = w * per < static_cast<int>(total) ? w * per : static_cast<int>(total);
    const int c1 = c0 + per < static_cast<int>(total) ? c0 + per : static_cast<int>(total);
    rank_range_write<BLOCK, E>(p, n, seg, sm.area, static_cast<int>(total), kk, c0, c1);
    TOPK_TRACE(11);
    return;
  }
  if (all_mode && nc <= kArea) {
    // Every in-range element, at its position: no counting needed.  Vectors whose wave range
    // holds no position of [lo, hi) are skipped as a whole (wave-uniform).
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int wpos = wslot(j) * EV;
      if (wpos >= hi || wpos + 64 * EV <= lo) continue;
      const u32 w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int e = 0; e < EV; ++e) {
        const int pos = vslot(j) * EV + e;
        const u32 b = E::element(w4, e);
        if (pos >= lo && pos < hi) sm.area[pos - lo] = E::pack(b, idx_base + static_cast<u32>(pos), inf);
      }
    }
    C = nc;
    __syncthreads();
  } else if (all_mode || overflow) {
    // ---- 4b. exact refinement (rare: ties or NaN-dominated rows overflow the LDS list).
    // Radix select over P = key << 17 | position17 among in-range elements with key prefix
    // <= T, until at most kArea values are <= the bound.  The chunk is re-read from memory for
    // each pass, so the registers of the fast path are not kept live for it.
    u64 prefix = 0, pmask = 0;
    int need = kc;
    for (int shift = E::kKeyBits + 16; shift >= 0; shift -= 8) {
      for (int i = tid; i < 256; i += BLOCK) sm.hist[i] = 0;
      __syncthreads();
      for_each_element([&](u32 b, int pos) {
        const u64 P = (static_cast<u64>(E::key(b, inf)) << 17) | static_cast<u32>(pos);
        if (E::prefix(b, inf) <= T && (P & pmask) == prefix) atomicAdd(&sm.hist[(P >> shift) & 255u], 1u);
      });
      __syncthreads();
      if (wid == 0) wave_find_bucket(sm.hist, need, sm.scal, lane);
      __syncthreads();
      const int b = sm.scal[0];
      const int before = sm.scal[1];
      const int cnt = sm.scal[2];
      need -= before;
      prefix |= static_cast<u64>(b) << shift;
      pmask |= 0xffull << shift;
      const int count_le = (kc - need) + cnt;
      if (count_le <= kArea) break;
    }
    const u64 bound = prefix | (~pmask & ((1ull << (E::kKeyBits + 17)) - 1));
    if (tid == 0) sm.scal[4] = 0;
    __syncthreads();
    for_each_element([&](u32 b, int pos) {
      const u64 P = (static_cast<u64>(E::key(b, inf)) << 17) | static_cast<u32>(pos);
      if (E::prefix(b, inf) <= T && P <= bound) {
        const int slot = atomicAdd(&sm.scal[4], 1);
        if (slot < kArea) sm.area[slot] = E::pack(b, idx_base + static_cast<u32>(pos), inf);
      }
    });
    __syncthreads();
    C = sm.scal[4];
    C = C < kArea ? C : kArea;
  }
  TOPK_TRACE(6);
  TOPK_TRACE_VALUE(14, C);
  TOPK_TRACE_VALUE(15, T);

  // ---- 5. multi-chunk segment: publish this chunk's list; the workgroup that merges goes
  // on to step 6 with the segment's lists gathered in LDS.
  int Mf = C;  // entries in sm.area that step 6 selects from
  if (Ws > 1) {
    const u64* src = sm.area;
    int M = C;
    if (C > p.cap_list) {
      const u64 bound = block_select_bound<BLOCK, E>(sm.area, C, kc, sm.hist, sm.scal, n);
      if (tid == 0) sm.scal[3] = 0;
      __syncthreads();
      for (int i = tid; i < C; i += BLOCK) {
        const u64 P = sm.area[i];
        if (P <= bound) {
          const int slot = atomicAdd(&sm.scal[3], 1);
          if (slot < p.kpad) sm.sel[slot] = P;
        }
      }
      __syncthreads();
      src = sm.sel;
      M = kc;
    }
    if (pair) {
      // Two chunks.  The first to arrive publishes its list (at most cap_list entries holding
      // its chunk's top kc) with every entry and the length word tagged for this call, and
      // returns without waiting for the stores.  The second gathers it into LDS after its
      // own list, polling until the length and every entry carry the tag, then clears the
      // consumed words (so a replay with the same epoch cannot take them for fresh ones) and
      // the ticket.
      const u64 etag = pair_entry_tag<E>(epoch);
    constexpr u64 kPairTagMask = pair_tag_mask<E>();
      const u32 ctag = pair_count_tag(epoch);
      if (!sm.scal[5]) {
        const int64_t my_id = static_cast<int64_t>(seg) * W + w;
        u64* dst = p.lists + my_id * p.cap_list;
        for (int i = tid; i < M; i += BLOCK) store_agent(dst + i, src[i] | etag);
        if (tid == 0) {
          store_agent(reinterpret_cast<u32*>(p.list_counts) + my_id, (ctag << 16) | static_cast<u32>(M));
        }
        TOPK_TRACE(8);
        return;
      }
      if (src != sm.area) {
        for (int i = tid; i < M; i += BLOCK) sm.area[i] = src[i];
      }
      const int64_t other = static_cast<int64_t>(seg) * W + (1 - w);
      u64* ol = p.lists + other * p.cap_list;
      u32* oc = reinterpret_cast<u32*>(p.list_counts) + other;
      const int cap = p.cap_list;
      const u32 want = (p.force_timeout & kForcePairPoll) ? (ctag ^ 1u) : ctag;
      int mp = 0;
      int seen = 0;  // workgroup-uniform count of waves that found a stale word so far
      u32 spin = 0;
      for (;; ++spin) {
        const u32 h = load_agent(oc);
        const u64 x = tid < cap ? load_agent(ol + tid) : 0ull;
        mp = static_cast<int>(h & 0xffffu);
        mp = mp < cap ? mp : cap;
        const bool bad = (h >> 16) != want || (tid < mp && (x & kPairTagMask) != etag);
        if (ballot(bad) && lane == 0) atomicAdd(&sm.scal[6], 1);
        __syncthreads();
        const int now = sm.scal[6];
        if (now == seen) {  // no wave saw a stale word: the list is complete
          if (tid < mp) sm.area[M + tid] = x & ~kPairTagMask;
          break;
        }
        seen = now;
        if (spin >= p.spin_limit) {  // gave up (the publisher has started, so only the test hook)
          mp = -1;
          break;
        }
        __syncthreads();  // every wave has read the count before the next round adds to it
        __builtin_amdgcn_s_sleep(1);
      }
      TOPK_TRACE_VALUE(13, spin + 1);
      if (tid < (mp < 0 ? cap : mp)) store_agent(ol + tid, 0ull);
      if (tid == 0) {
        store_agent(oc, 0u);
        store_agent(p.tickets + seg, 0ull);
      }
      if (mp < 0) {
        give_up_row<BLOCK, E>(p, seg, nullptr);
        return;
      }
      if (tid == 0) p.status[seg] = kStatusOk;
      Mf = M + mp;
    } else {
      // Three or more chunks: every workgroup publishes, the last to arrive merges.
      const int64_t list_id = static_cast<int64_t>(seg) * W + w;
      u64* my_list = p.lists + list_id * p.cap_list;
      for (int i = tid; i < M; i += BLOCK) {
        __hip_atomic_store(my_list + i, src[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (tid == 0) __hip_atomic_store(p.list_counts + list_id, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      wait_vector_memory();
      __syncthreads();
      TOPK_TRACE(8);
      if (tid == 0) sm.scal[5] = arrive_last(p.tickets + seg, p.epoch, Ws) ? 1 : 0;
      __syncthreads();
      TOPK_TRACE(9);
      if (!sm.scal[5]) return;
      if (tid == 0) p.status[seg] = kStatusOk;

      int total = 0;
      for (int c = 0; c < Ws; ++c) {
        const int64_t id = static_cast<int64_t>(seg) * W + c;
        int cnt = __hip_atomic_load(p.list_counts + id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        cnt = cnt < 0 ? 0 : (cnt > p.cap_list ? p.cap_list : cnt);
        if (total + cnt > kArea) cnt = kArea - total;
        const u64* lst = p.lists + id * p.cap_list;
        for (int i = tid; i < cnt; i += BLOCK) {
          sm.area[total + i] = __hip_atomic_load(lst + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        total += cnt;
      }
      Mf = total;
    }
    __syncthreads();
    TOPK_TRACE(10);
  }

  // ---- 6. select and write the segment's row
  finalize_segment<BLOCK, E>(p, sm, Mf, kk, n, seg);
  TOPK_TRACE(11);
}

// ------------------------------------------------------------------------------ long segments

// Loads vectors J0 .. J0 + NV - 1 of chunk cb (positions [lo, hi) valid) as the main kernel
// loads its chunk: nontemporal 16-byte buffer loads, positions outside [lo, hi) set to the NaN
// filler.
template <int BLOCK, int NV, class E>
__device__ __forceinline__ void load_chunk(const TopkParams& p, int64_t cb, int lo, int hi, int J0, uint4 (&v)[NV]) {
  constexpr int EV = E::kPerVec;
  const int tid = threadIdx.x;
  const unsigned char* cptr = reinterpret_cast<const unsigned char*>(p.base) + cb * E::kBytes;
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<unsigned char*>(cptr), static_cast<short>(0), ((hi + EV - 1) & ~(EV - 1)) * E::kBytes,
      kBufferWord3);
#pragma unroll
  for (int jj = 0; jj < NV; ++jj) {
    const u32x4_t t =
        __builtin_amdgcn_raw_buffer_load_b128(rsrc, tid * 16, (J0 + jj) * BLOCK * 16, kCachePolicyNT);
    v[jj] = make_uint4(t.x, t.y, t.z, t.w);
  }
#pragma unroll
  for (int jj = 0; jj < NV; ++jj) {
    const int j = J0 + jj;
    if ((j == 0 && lo > 0) || (j + 1) * BLOCK * EV > hi) {
      const int pos = (j * BLOCK + tid) * EV;
      if (pos < lo || pos + EV > hi) {
        u32 w4[4] = {v[jj].x, v[jj].y, v[jj].z, v[jj].w};
#pragma unroll
        for (int e = 0; e < EV; ++e) {
          if (pos + e < lo || pos + e >= hi) E::fill(w4, e);
        }
        v[jj] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
      }
    }
  }
}

// Key prefix of the thread's best element over its VPT vectors (a NaN filler only if the thread
// holds nothing better), as in the main kernel's step 2.
template <int VPT, class E>
__device__ __forceinline__ u32 thread_best_key(const uint4 (&v)[VPT], u32 inf) {
  int m1, m2;
  if constexpr (E::kBytes == 2) {
    int mx = vec_gmax(as_s2(vec_max2(v[0])));
#pragma unroll
    for (int j = 1; j < VPT; ++j) {
      const int t = vec_gmax(as_s2(vec_max2(v[j])));
      mx = mx > t ? mx : t;
    }
    m1 = mx;
    m2 = 32767;
    if (ballot(m1 < 0)) {
      short2_t mn = as_s2(vec_min2(v[0]));
#pragma unroll
      for (int j = 1; j < VPT; ++j) mn = __builtin_elementwise_min(mn, as_s2(vec_min2(v[j])));
      m2 = mn.x < mn.y ? mn.x : mn.y;
    }
  } else {
    int mx = vec_max4_i32(v[0]);
#pragma unroll
    for (int j = 1; j < VPT; ++j) {
      const int t = vec_max4_i32(v[j]);
      mx = mx > t ? mx : t;
    }
    m1 = mx;
    m2 = 0x7fffffff;
    if (ballot(m1 < 0)) {
      int mn = vec_min4_i32(v[0]);
#pragma unroll
      for (int j = 1; j < VPT; ++j) {
        const int t = vec_min4_i32(v[j]);
        mn = mn < t ? mn : t;
      }
      m2 = mn;
    }
  }
  const u32 bits = static_cast<u32>(m1 >= 0 ? m1 : m2) & (E::kBytes == 2 ? 0xffffu : 0xffffffffu);
  return E::prefix(bits, inf);
}

// Segments longer than one co-resident grid of single-chunk workgroups covers: p.group
// workgroups per segment (grid seg_num * group), workgroup w taking chunks w, w + group, ...
// of 1024 threads x 16 vectors.  The steps are those of the cooperative path: the thread bests
// of every chunk a workgroup takes go into its LDS histograms (high byte, and 32-key bins),
// which are summed over the segment in one meeting; T is the last key of the fine bin holding
// the kk-th best; every chunk is read again and its elements with key prefix <= T are listed;
// the lists meet in one gather and every workgroup ranks a share.  An exact radix refinement
// over (key, index32) takes over when the lists overflow.  With one workgroup per segment
// (many segments) nothing is exchanged: the histograms and the list stay in LDS, and the
// workgroup selects and ranks its segment's list itself.  Every cross-workgroup word carries
// the per-call token, every wait is bounded, and the segment's status word records a give-up,
// as on the cooperative path.
template <class E>
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4)))
long_segment_kernel(TopkParams p) {
  constexpr int BLOCK = 1024;
  constexpr int VPT = 16;
  constexpr int EV = E::kPerVec;
  constexpr int CH = BLOCK * VPT * EV;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const Smem sm = carve_smem(smem_raw, p.kpad);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int G = p.group;
  const int seg = static_cast<int>(blockIdx.x) / G;
  const int w = static_cast<int>(blockIdx.x) - seg * G;
  const int k = p.k;
  const u32 inf = p.inf_bits;

  int64_t s0, s1;
  if (p.offsets) {
    s0 = p.offsets[seg];
    s1 = p.offsets[seg + 1];
    if (s1 < s0) s1 = s0;
  } else {
    s0 = static_cast<int64_t>(seg) * p.seg_len;
    s1 = s0 + p.seg_len;
  }
  s0 += p.elem0;
  s1 += p.elem0;
  const int64_t n = s1 - s0;
  const int64_t a0 = s0 & ~static_cast<int64_t>(EV - 1);
  const int64_t Ws64 = n > 0 ? (s1 - a0 + CH - 1) / CH : 0;
  if (n <= 0 || n > p.max_len || Ws64 > p.chunks_per_seg) {
    if (w == 0) {
      for (int r = tid; r < k; r += BLOCK) write_pad<E>(p, static_cast<int64_t>(seg) * k + r);
      if (tid == 0) store_agent(p.status + seg, kStatusOk);
    }
    return;
  }
  const int Ws = static_cast<int>(Ws64);
  const int arrivals = Ws < G ? Ws : G;  // workgroups of the segment that take chunks
  if (w >= arrivals) return;
  const bool solo = arrivals == 1;
  const int kk = n < k ? static_cast<int>(n) : k;
  // chunk c of the segment: base cb (16-byte aligned), valid positions [lo, hi)
  auto chunk_range = [&](int c, int64_t& cb, int& lo, int& hi) {
    cb = a0 + static_cast<int64_t>(c) * CH;
    const int64_t c0 = s0 > cb ? s0 : cb;
    const int64_t c1 = s1 < cb + CH ? s1 : cb + CH;
    lo = static_cast<int>(c0 - cb);
    hi = static_cast<int>(c1 - cb);
  };
  // Calls fn(raw bits, segment index) for every element of every chunk this workgroup takes,
  // re-read with plain loads (the refinement passes).
  auto for_each_element = [&](auto&& fn) {
    for (int c = w; c < Ws; c += arrivals) {
      int64_t cb;
      int lo, hi;
      chunk_range(c, cb, lo, hi);
      const unsigned char* cptr = reinterpret_cast<const unsigned char*>(p.base) + cb * E::kBytes;
      const u32 idx_base = static_cast<u32>(cb - s0);
#pragma unroll 1
      for (int j = 0; j < VPT; ++j) {
        const int pos0 = (j * BLOCK + tid) * EV;
        if (pos0 < hi && pos0 + EV > lo) {
          const uint4 x = *reinterpret_cast<const uint4*>(cptr + static_cast<u32>(pos0) * E::kBytes);
          const u32 w4[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
          for (int e = 0; e < EV; ++e) {
            const int pos = pos0 + e;
            if (pos >= lo && pos < hi) fn(E::element(w4, e), idx_base + static_cast<u32>(pos));
          }
        }
      }
    }
  };

  // Call token, status reset and (workgroup 0 of a shared segment) the global histograms'
  // clear, as on the cooperative path.
  const u64 epoch = p.epoch;
  u64 token = epoch;
  const GroupWs g = group_ws(p, seg, G);
  if (tid == 0) {
    if (!solo) token = call_token(epoch, load_agent(g.gen));
    reinterpret_cast<u64*>(sm.wcnt)[0] = token;
    if (w == 0) store_agent(p.status + seg, kStatusOk);
  }
  if (!solo && w == 0) {
    for (int i = tid; i < kGroupCopies * 256; i += BLOCK) store_agent(g.hist + i, 0u);
    for (int i = tid; i < kFineCopies * kFineBins; i += BLOCK) store_agent(g.fine + i, 0u);
    for (int i = tid; i < kRefineDigits * 256; i += BLOCK) store_agent(g.rhist + i, 0u);
    wait_vector_memory();
    __syncthreads();
    if (tid == 0) store_agent(g.flag, ((token & kTagMask) << 20) | 1u);
  }
  u32* fine = reinterpret_cast<u32*>(sm.area);  // 32-key bins, in the (unused) candidate area
  for (int i = tid; i < 256; i += BLOCK) sm.hist[i] = 0;
  for (int i = tid; i < kFineBins; i += BLOCK) fine[i] = 0;
  __syncthreads();
  token = reinterpret_cast<const u64*>(sm.wcnt)[0];
  const u64 tag = token & kTagMask;

  // ---- A. the thread bests of every chunk this workgroup takes, into the LDS histograms
  for (int c = w; c < Ws; c += arrivals) {
    int64_t cb;
    int lo, hi;
    chunk_range(c, cb, lo, hi);
    u32 bk = 0xffffffffu;
#pragma unroll 1
    for (int J0 = 0; J0 < VPT; J0 += VPT / 2) {  // half a chunk at a time (register pressure)
      uint4 v[VPT / 2];
      load_chunk<BLOCK, VPT / 2, E>(p, cb, lo, hi, J0, v);
      const u32 hk = thread_best_key<VPT / 2, E>(v, inf);
      bk = hk < bk ? hk : bk;
    }
    atomicAdd(&sm.hist[bk >> 8], 1u);
    atomicAdd(&fine[bk >> 5], 1u);
  }
  __syncthreads();
  if (!solo) {
    int late = 0;
    if (tid == 0) {  // the global histograms are cleared
      const u32 want = (p.force_timeout & kForceFlagWait) ? 2u : 1u;
      late = 1;
      for (u32 spin = 0; spin < p.spin_limit; ++spin) {
        if (tagged_value(load_agent(g.flag), tag) == want) {
          late = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    }
    if (__syncthreads_or(late)) {
      give_up_row<BLOCK, E>(p, seg, g.gen);
      return;
    }
    for (int i = tid; i < kFineBins; i += BLOCK) {
      const u32 c = fine[i];
      if (c) {
        __hip_atomic_fetch_add(g.fine + (w % kFineCopies) * kFineBins + i, c, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    const u64 expect = (p.force_timeout & kForceBarrier) ? (token ^ 1u) : token;
    if (!group_histogram<BLOCK>(sm.hist, g.hist, sm.stage, g.arrive, token, expect, w, arrivals, p.spin_limit)) {
      give_up_row<BLOCK, E>(p, seg, g.gen);
      return;
    }
    if (w == 0 && tid == 0) __hip_atomic_fetch_add(g.gen, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // T: the last key of the 32-key bin holding the kk-th smallest thread best (at least kk real
  // elements are at or below it).
  if (wid == 0) wave_find_bucket(sm.hist, kk, sm.scal + 8, lane);
  __syncthreads();
  const u32 b1 = static_cast<u32>(sm.scal[8]);
  if (tid < 8 * kFineCopies) {  // the 8 fine bins of bucket b1, copy by copy
    const int q = tid >> 3;
    sm.stage[tid] = solo ? (q == 0 ? fine[b1 * 8 + (tid & 7)] : 0u)
                         : load_agent(g.fine + q * kFineBins + b1 * 8 + (tid & 7));
  }
  __syncthreads();
  if (wid == 0) {
    u32 c = 0;
    if (lane < 8) {
#pragma unroll
      for (int q = 0; q < kFineCopies; ++q) c += sm.stage[q * 8 + lane];
    }
    const u32 incl = wave_inclusive_scan(c);
    const u32 rest = static_cast<u32>(kk - sm.scal[9]);
    const u64 m = ballot(lane < 8 && incl >= rest);
    if (lane == static_cast<int>(__builtin_ctzll(m))) sm.scal[12] = lane;
  }
  if (tid == 0) sm.scal[4] = 0;
  __syncthreads();
  const u32 T = (((b1 << 3) | static_cast<u32>(sm.scal[12])) << 5) | 31u;

  // ---- B. every chunk again: its elements with key prefix <= T, one ballot per element
  // position, into per-wave LDS regions that one atomic per wave and chunk places in the list.
  if (T == 0xffffu) {
    if (tid == 0) sm.scal[4] = kArea + 1;  // no usable threshold: the refinement decides
  } else {
    constexpr int RC = kStageWords / 2;
    u64* region = reinterpret_cast<u64*>(sm.stage + wid * kStageWords);
    for (int c = w; c < Ws; c += arrivals) {
      int64_t cb;
      int lo, hi;
      chunk_range(c, cb, lo, hi);
      const u32 idx_base = static_cast<u32>(cb - s0);
      u32 wcount = 0;  // wave-uniform
#pragma unroll 1
      for (int J0 = 0; J0 < VPT; J0 += VPT / 2) {  // half a chunk at a time (register pressure)
        uint4 v[VPT / 2];
        load_chunk<BLOCK, VPT / 2, E>(p, cb, lo, hi, J0, v);
#pragma unroll
        for (int jj = 0; jj < VPT / 2; ++jj) {
          const u32 w4[4] = {v[jj].x, v[jj].y, v[jj].z, v[jj].w};
#pragma unroll
          for (int e = 0; e < EV; ++e) {
            const u32 b = E::element(w4, e);  // positions outside [lo, hi) hold the NaN filler
            const bool h = E::prefix(b, inf) <= T;
            const u64 m = ballot(h);
            if (m) {
              if (h) {
                const u32 slot = wcount + mbcnt(m);
                if (slot < static_cast<u32>(RC))
                  region[slot] = E::pack(b, idx_base + static_cast<u32>(((J0 + jj) * BLOCK + tid) * EV + e), inf);
              }
              wcount += static_cast<u32>(__popcll(m));
            }
          }
        }
      }
      const u32 amount = wcount > static_cast<u32>(RC) ? static_cast<u32>(kArea) + 1u : wcount;
      if (amount) {
        wave_lds_sync();
        u32 base = 0;
        if (lane == 0) base = atomicAdd(reinterpret_cast<u32*>(&sm.scal[4]), amount);
        base = __builtin_amdgcn_readfirstlane(base);
        if (wcount <= static_cast<u32>(RC)) {
          for (u32 i = lane; i < wcount; i += 64) {
            if (base + i < static_cast<u32>(kArea)) sm.area[base + i] = region[i];
          }
        }
        wave_lds_sync();  // the region is reused by the next chunk
      }
    }
  }
  __syncthreads();
  const int C = sm.scal[4];

  // ---- C. the segment's list: every workgroup's list gathered (or the solo list in place);
  // the refinement when one overflowed or the whole list would not fit the gather.
  int* cnt = reinterpret_cast<int*>(sm.hist);   // [256] list lengths of the workgroups
  int* pre = reinterpret_cast<int*>(sm.hist2);  // [256] their exclusive prefix sums
  u64* mylist = g.lists + static_cast<size_t>(w) * kCandArea;
  u32 total;
  if (solo) {
    total = C > kArea ? kAbsent : static_cast<u32>(C);
  } else {
    const u32 contrib = C > kArea ? static_cast<u32>(kCandArea) + 1u : static_cast<u32>(C);
    if (contrib <= static_cast<u32>(kCandArea)) {
      for (u32 i = tid; i < contrib; i += BLOCK) store_agent(mylist + i, sm.area[i]);
    }
    wait_vector_memory();  // the list is complete before its length announces it
    __syncthreads();
    if (tid == 0) store_agent(g.counts + w, (tag << 20) | contrib);
    const u64 want = (p.force_timeout & kForceCollect) ? (tag ^ 1u) : tag;
    total = group_collect<BLOCK>(g.counts, g.lists, want, arrivals, sm.area, cnt, pre, sm.scal + 20, p.spin_limit);
    if (total == kGaveUp) {
      give_up_row<BLOCK, E>(p, seg, g.gen);
      return;
    }
  }
  if (total == kAbsent) {
    // Exact radix refinement of Q = key << 32 | index32 among the elements with key prefix
    // <= T (one histogram per 8-bit digit, summed over the segment), until at most kCandArea
    // elements are at or below the bound.
    u64 prefix = 0, pmask = 0;
    int rneed = kk;
    int pass = 0;
    constexpr u64 kQMask = E::kKeyBits == 32 ? ~0ull : ((1ull << (32 + E::kKeyBits)) - 1);
    for (int shift = E::kKeyBits + 24; shift >= 0; shift -= 8, ++pass) {
      for (int i = tid; i < 256; i += BLOCK) sm.hist[i] = 0;
      __syncthreads();
      for_each_element([&](u32 b, u32 idx) {
        const u64 Q = (static_cast<u64>(E::key(b, inf)) << 32) | idx;
        if (E::prefix(b, inf) <= T && (Q & pmask) == prefix) atomicAdd(&sm.hist[(Q >> shift) & 255u], 1u);
      });
      __syncthreads();
      if (!solo && !group_histogram_single<BLOCK>(sm.hist, g.rhist + pass * 256, g.arrive + (3 + pass) * G, token,
                                                  w, arrivals, p.spin_limit)) {
        give_up_row<BLOCK, E>(p, seg, g.gen);
        return;
      }
      if (wid == 0) wave_find_bucket(sm.hist, rneed, sm.scal, lane);
      __syncthreads();
      const int b = sm.scal[0];
      const int before = sm.scal[1];
      const int cnt_b = sm.scal[2];
      __syncthreads();
      rneed -= before;
      prefix |= static_cast<u64>(b) << shift;
      pmask |= 0xffull << shift;
      if ((kk - rneed) + cnt_b <= kCandArea) break;
    }
    const u64 bound = prefix | (~pmask & kQMask);
    if (tid == 0) sm.scal[4] = 0;
    __syncthreads();
    for_each_element([&](u32 b, u32 idx) {
      const u64 Q = (static_cast<u64>(E::key(b, inf)) << 32) | idx;
      if (E::prefix(b, inf) <= T && Q <= bound) {
        const int slot = atomicAdd(&sm.scal[4], 1);
        if (slot < kArea) sm.area[slot] = E::pack(b, idx, inf);
      }
    });
    __syncthreads();
    const u32 c2 = static_cast<u32>(sm.scal[4] < kArea ? sm.scal[4] : kArea);
    if (solo) {
      total = c2;
    } else {
      for (u32 i = tid; i < c2; i += BLOCK) store_agent(mylist + i, sm.area[i]);
      wait_vector_memory();
      __syncthreads();
      if (tid == 0) store_agent(g.counts + G + w, (tag << 20) | c2);
      total = group_collect<BLOCK>(g.counts + G, g.lists, tag, arrivals, sm.area, cnt, pre, sm.scal + 20,
                                   p.spin_limit);
      if (total == kGaveUp) {
        give_up_row<BLOCK, E>(p, seg, g.gen);
        return;
      }
      if (total == kAbsent) total = 0;  // cannot happen: at most kCandArea elements are <= bound
    }
  }

  // ---- D. ranks and the output row.  Shared segments rank a share of the list per workgroup
  // (workgroup 0 also writes the pads); a solo workgroup selects the kk best (radix select)
  // when the list is longer than a workgroup's threads and ranks them in sorted runs.
  if (w == 0) {
    for (int r = kk + tid; r < k; r += BLOCK) write_pad<E>(p, static_cast<int64_t>(seg) * k + r);
  }
  const int M = static_cast<int>(total);
  if (!solo) {
    const int per = (M + arrivals - 1) / arrivals;
    const int r0 = w * per < M ? w * per : M;
    const int r1 = r0 + per < M ? r0 + per : M;
    rank_range_write<BLOCK, E>(p, n, seg, sm.area, M, kk, r0, r1);
    return;
  }
  u64* list = sm.area;
  int Ml = M;
  if (M > BLOCK) {
    const u64 bound = block_select_bound<BLOCK, E>(sm.area, M, kk, sm.hist, sm.scal, n);
    if (tid == 0) sm.scal[3] = 0;
    __syncthreads();
    for (int i = tid; i < M; i += BLOCK) {
      const u64 P = sm.area[i];
      if (P <= bound) {
        const int slot = atomicAdd(&sm.scal[3], 1);
        if (slot < p.kpad) sm.sel[slot] = P;
      }
    }
    __syncthreads();
    list = sm.sel;
    Ml = kk;
  }
  sort_rank_write<BLOCK, E>(p, n, seg, list, Ml, kk, nullptr);
}

// Device attributes the launches use, cached per device: CUs, LDS per CU, LDS per workgroup.
struct DeviceInfo {
  int cus;
  int lds_per_cu;
  int lds_per_block;
};
DeviceInfo device_info() {
  static std::atomic<int> cached[64][3];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return DeviceInfo{0, 0, 0};
  if (dev < 64 && cached[dev][0].load(std::memory_order_relaxed) > 0) {
    return DeviceInfo{cached[dev][0].load(std::memory_order_relaxed), cached[dev][1].load(std::memory_order_relaxed),
                      cached[dev][2].load(std::memory_order_relaxed)};
  }
  DeviceInfo d{0, 0, 0};
  if (hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return DeviceInfo{0, 0, 0};
  if (hipDeviceGetAttribute(&d.lds_per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess ||
      hipDeviceGetAttribute(&d.lds_per_block, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) {
    d.lds_per_cu = d.lds_per_block = 0;  // no spreading (spread_lds)
  }
  if (dev < 64) {
    cached[dev][1].store(d.lds_per_cu, std::memory_order_relaxed);
    cached[dev][2].store(d.lds_per_block, std::memory_order_relaxed);
    cached[dev][0].store(d.cus, std::memory_order_relaxed);
  }
  return d;
}

int device_cu_count() { return device_info().cus; }

// Dynamic LDS of a launch of 1024-thread workgroups: when the grid fits the CUs, more than half
// a CU's LDS, so that the dispatcher gives every workgroup a CU of its own.  (A kernel of at
// most 64 VGPRs fits twice on a CU: two workgroups placed together share one CU's memory
// pipeline, about 64 KB of loads in flight, while other CUs stay idle.)
unsigned spread_lds(size_t lds_bytes, int64_t grid) {
  const DeviceInfo d = device_info();
  if (d.cus <= 0 || grid > d.cus || d.lds_per_cu <= 0) return static_cast<unsigned>(lds_bytes);
  const size_t want = static_cast<size_t>(d.lds_per_cu) / 2 + 256;
  if (want > static_cast<size_t>(d.lds_per_block)) return static_cast<unsigned>(lds_bytes);
  return static_cast<unsigned>(lds_bytes > want ? lds_bytes : want);
}

template <int BLOCK, int VPT, class E>
int launch_shape(const Plan& plan, const TopkParams& params, hipStream_t stream) {
  const int64_t groups = static_cast<int64_t>(params.seg_num) * params.chunks_per_seg;
  const dim3 grid(static_cast<unsigned>(groups));
  const unsigned lds = BLOCK == 1024 ? spread_lds(plan.lds_bytes, groups) : static_cast<unsigned>(plan.lds_bytes);
  // Chunks that can be short (all positions in each thread's first vector, at most 4 * EV * k
  // elements): segmented input, or fixed-length rows that short.
  const int64_t ev = E::kPerVec;
  const bool short_chunks = params.offsets != nullptr ||
                            (params.seg_len + ev - 1 <= BLOCK * ev && params.seg_len <= 4 * ev * params.k);
  if (short_chunks) {
    hipLaunchKernelGGL((segmented_topk_kernel<BLOCK, VPT, false, E, true>), grid, dim3(BLOCK), lds, stream,
                       params);
    return static_cast<int>(hipGetLastError());
  }
  hipLaunchKernelGGL((segmented_topk_kernel<BLOCK, VPT, false, E>), grid, dim3(BLOCK), lds, stream, params);
  return static_cast<int>(hipGetLastError());
}

// Launch of the cooperative path (1024 threads, 16 or 8 vectors each).  Its workgroups wait
// for each other, so all of them must be resident at once: one 1024-thread workgroup fits every
// CU, and the grid is refused (hipErrorCooperativeLaunchTooLarge) when it has more workgroups
// than the device has CUs.
// Within that bound an ordinary launch places every workgroup immediately (kernels of other
// streams only delay the placement; they do not wait for this one), and it costs far less
// than hipLaunchCooperativeKernel.  BATCH_TOPK_AMD_COOPERATIVE_LAUNCH=1 selects the runtime's
// cooperative launch, which checks co-residency itself.
bool formal_cooperative_launch() {
  static const bool on = [] {
    const char* e = std::getenv("BATCH_TOPK_AMD_COOPERATIVE_LAUNCH");
    return e != nullptr && e[0] == '1';
  }();
  return on;
}

template <int VPT, class E>
int launch_cooperative(const Plan& plan, TopkParams params, hipStream_t stream) {
  const int64_t groups = static_cast<int64_t>(params.seg_num) * params.chunks_per_seg;
  if (groups > device_cu_count()) return static_cast<int>(hipErrorCooperativeLaunchTooLarge);
  const dim3 grid(static_cast<unsigned>(groups));
  const unsigned lds = spread_lds(plan.lds_bytes, groups);
  if (formal_cooperative_launch()) {
    void* args[] = {&params};
    const hipError_t e = hipLaunchCooperativeKernel(
        reinterpret_cast<const void*>(&segmented_topk_kernel<1024, VPT, true, E>), grid, dim3(1024), args, lds,
        stream);
    if (e != hipSuccess) return static_cast<int>(e);
  } else {
    hipLaunchKernelGGL((segmented_topk_kernel<1024, VPT, true, E>), grid, dim3(1024), lds, stream, params);
  }
  return static_cast<int>(hipGetLastError());
}

// Launch of the long-segment path: seg_num * group workgroups of 1024 threads.  With several
// workgroups per segment they wait for each other, so (as on the cooperative path) the grid
// must fit the CUs; one workgroup per segment waits for nothing.
template <class E>
int launch_long(const Plan& plan, const TopkParams& params, hipStream_t stream) {
  const int64_t groups = static_cast<int64_t>(params.seg_num) * params.group;
  if (params.group > 1 && groups > device_cu_count()) return static_cast<int>(hipErrorCooperativeLaunchTooLarge);
  hipLaunchKernelGGL((long_segment_kernel<E>), dim3(static_cast<unsigned>(groups)), dim3(1024),
                     spread_lds(plan.lds_bytes, groups), stream, params);
  return static_cast<int>(hipGetLastError());
}

// The instantiation for the plan's workgroup shape and element format.
template <class E>
int launch_format(const Plan& plan, const TopkParams& params, hipStream_t s) {
  const int b = plan.shape.block;
  const int vpt = plan.shape.vpt;
  if (plan.group > 0) {
    if (b != 1024 || vpt != 16) return static_cast<int>(hipErrorInvalidValue);
    return launch_long<E>(plan, params, s);
  }
  if (plan.cooperative) {
    if (b == 1024 && vpt == 16) return launch_cooperative<16, E>(plan, params, s);
    if (b == 1024 && vpt == 8) return launch_cooperative<8, E>(plan, params, s);
    return static_cast<int>(hipErrorInvalidValue);
  }
  if (b == 256 && vpt == 2) return launch_shape<256, 2, E>(plan, params, s);
  if (b == 256 && vpt == 4) return launch_shape<256, 4, E>(plan, params, s);
  if (b == 256 && vpt == 8) return launch_shape<256, 8, E>(plan, params, s);
  if (b == 256 && vpt == 16) return launch_shape<256, 16, E>(plan, params, s);
  if (b == 512 && vpt == 2) return launch_shape<512, 2, E>(plan, params, s);
  if (b == 512 && vpt == 4) return launch_shape<512, 4, E>(plan, params, s);
  if (b == 512 && vpt == 8) return launch_shape<512, 8, E>(plan, params, s);
  if (b == 512 && vpt == 16) return launch_shape<512, 16, E>(plan, params, s);
  if (b == 1024 && vpt == 2) return launch_shape<1024, 2, E>(plan, params, s);
  if (b == 1024 && vpt == 4) return launch_shape<1024, 4, E>(plan, params, s);
  if (b == 1024 && vpt == 8) return launch_shape<1024, 8, E>(plan, params, s);
  if (b == 1024 && vpt == 16) return launch_shape<1024, 16, E>(plan, params, s);
  return static_cast<int>(hipErrorInvalidValue);
}

}  // namespace

int launch_segmented_topk(const Plan& plan, const TopkParams& params, void* stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return params.elem_bytes == 4 ? launch_format<Elem32>(plan, params, s) : launch_format<Elem16>(plan, params, s);
}

}  // namespace radix_topk_amd

#ifdef TOPK_PHASE_TRACE
// Profiling build only: copies the phase tables to host buffers (kMaxWorkgroups x 16 words each
// for the workgroup tables, x 16 x 16 for the wave table), or zeroes them.
extern "C" int radix_topk_trace_fetch(void* clock, void* real, void* wave) {
  using namespace radix_topk_amd_trace;
  hipError_t e = hipMemcpyFromSymbol(clock, HIP_SYMBOL(g_clock), sizeof(g_clock));
  if (e == hipSuccess) e = hipMemcpyFromSymbol(real, HIP_SYMBOL(g_real), sizeof(g_real));
  if (e == hipSuccess) e = hipMemcpyFromSymbol(wave, HIP_SYMBOL(g_wave), sizeof(g_wave));
  return static_cast<int>(e);
}
extern "C" int radix_topk_trace_clear() {
  using namespace radix_topk_amd_trace;
  static unsigned long long zeros[kMaxWorkgroups * 16 * 16];
  hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(g_clock), zeros, sizeof(g_clock));
  if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(g_real), zeros, sizeof(g_real));
  if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(g_wave), zeros, sizeof(g_wave));
  return static_cast<int>(e);
}
#endif
