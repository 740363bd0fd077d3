// Fused segmented fp16 top-k for gfx950 (MI355X).
//
// One workgroup owns one chunk (block * vpt * 8 elements) of one segment and reads it from
// HBM exactly once, with 16-byte loads, into registers.  Everything after the load runs on
// registers and LDS:
//
//   1. thread best     packed int16 max/min over the raw fp16 bits (v_pk_max_i16 /
//                      v_pk_min_i16, one op per two elements).  The int16 max is the best
//                      non-negative-sign element, the int16 min the best negative-sign one;
//                      whichever applies is a real element of the thread (or, for a NaN,
//                      a worse one), which is all the threshold step needs.
//   2. threshold       each wave takes the ceil(kc / waves)-th smallest descending key of
//                      its lanes' bests with a 16-step ballot radix select (no LDS, no
//                      atomics); T = the largest of the wave results.  At least kc real
//                      elements have key <= T, so every element of the chunk's top kc does.
//   3. compaction      one pass over the registers with a single integer compare per
//                      element; hits are appended to an LDS list (wave-aggregated atomic
//                      slot) as packed (key16 << 32 | segment index).  If the list would
//                      overflow (ties, all-equal rows), an exact 4-digit radix refinement
//                      over (key16, position16) on the registers shrinks it first.
//   4. selection       an LDS radix select over the packed 48-bit (key, index) values finds
//                      the exact k-th entry, then a rank sort (or, for <= 64 entries, a
//                      wave64 register bitonic) orders the survivors.
//   5. output          values are re-read raw from the input at the selected index.
//
// Segments longer than one chunk are split over W workgroups.  Each publishes its list to
// the workspace, and the last to arrive (an epoch-tagged arrival counter, so the workspace
// needs no initialisation) merges the lists with step 4.
//
// Ordering contract (reference include/batch_topk_types.cuh:70-82,100-113 and
// include/type_codec.cuh:9-38): ascending (desc_key, index), where desc_key maps every NaN
// to 0xFFFF, +-0 to 0x7FFF, and is strictly decreasing in value otherwise.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "topk_common.hpp"

namespace radix_topk_amd {
namespace {

using u32 = uint32_t;
using u64 = unsigned long long;
typedef short short2_t __attribute__((ext_vector_type(2)));

constexpr u64 kMask48 = 0xFFFFFFFFFFFFull;
constexpr u32 kFillWord = 0xFFFFFFFFu;  // two negative NaNs: never a candidate, never a best

// ------------------------------------------------------------------------------ codec

// Descending order-preserving key of raw fp16 bits (reference include/type_codec.cuh:13-38):
// NaN -> 0xFFFF, +-0 -> 0x7FFF, negative -> bits, positive -> bits ^ 0x7FFF.
__device__ __forceinline__ u32 desc_key(u32 b) {
  const u32 mag = b & 0x7fffu;
  u32 key = (b & 0x8000u) ? b : (b ^ 0x7fffu);
  key = (mag == 0u) ? 0x7fffu : key;
  key = (mag > 0x7c00u) ? 0xffffu : key;
  return key;
}

// ------------------------------------------------------------------------------ wave64 helpers

__device__ __forceinline__ u64 ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

__device__ __forceinline__ u32 mbcnt(u64 m) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<u32>(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<u32>(m), 0u));
}

__device__ __forceinline__ u32 shfl_u32(u32 x, int src_lane) {
  return static_cast<u32>(__builtin_amdgcn_ds_bpermute(src_lane << 2, static_cast<int>(x)));
}

__device__ __forceinline__ u64 shfl_xor_u64(u64 x, int mask, int lane) {
  const int src = (lane ^ mask) << 2;
  const u32 lo = static_cast<u32>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(static_cast<u32>(x))));
  const u32 hi = static_cast<u32>(__builtin_amdgcn_ds_bpermute(src, static_cast<int>(static_cast<u32>(x >> 32))));
  return (static_cast<u64>(hi) << 32) | lo;
}

__device__ __forceinline__ u32 wave_inclusive_scan(u32 x, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const u32 y = shfl_u32(x, lane >= d ? lane - d : lane);
    if (lane >= d) x += y;
  }
  return x;
}

// kth (1-based, wave-uniform, 1..64) smallest 16-bit key across the 64 lanes of a wave:
// MSB-first binary radix select with ballots.  Pure SALU bookkeeping per bit.
__device__ __forceinline__ u32 wave_kth_smallest16(u32 key, int kth) {
  u64 run = ~0ull;
  u32 prefix = 0;
#pragma unroll
  for (int bit = 15; bit >= 0; --bit) {
    const u64 zeros = ballot(((key >> bit) & 1u) == 0u) & run;
    const int cz = __popcll(zeros);
    if (kth <= cz) {
      run = zeros;
    } else {
      kth -= cz;
      run &= ~zeros;
      prefix |= 1u << bit;
    }
  }
  return prefix;
}

// Ascending bitonic sort of one u64 per lane across a wave64.
__device__ __forceinline__ u64 wave_bitonic_sort64(u64 x, int lane) {
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const u64 o = shfl_xor_u64(x, stride, lane);
      const bool ascending = (lane & size) == 0;
      const bool lower = (lane & stride) == 0;
      const u64 mn = x < o ? x : o;
      const u64 mx = x < o ? o : x;
      x = (lower == ascending) ? mn : mx;
    }
  }
  return x;
}

// ------------------------------------------------------------------------------ LDS layout

struct Smem {
  u32* hist;    // [256]
  int* scal;    // [16]
  u32* wave_t;  // [16]
  u64* cand;    // [cand_area]
  u64* sel;     // [kpad]
  int* rank;    // [kpad]
};

__device__ __forceinline__ Smem carve_smem(unsigned char* smem, int cand_area, int kpad) {
  Smem s;
  s.hist = reinterpret_cast<u32*>(smem);
  s.scal = reinterpret_cast<int*>(s.hist + 256);
  s.wave_t = reinterpret_cast<u32*>(s.scal + 16);
  s.cand = reinterpret_cast<u64*>(s.wave_t + 16);
  s.sel = s.cand + cand_area;
  s.rank = reinterpret_cast<int*>(s.sel + kpad);
  return s;
}

// Wave 0: find the histogram bucket holding the need-th (1-based) entry.  Writes
// scal[0] = bucket, scal[1] = entries in earlier buckets, scal[2] = entries in the bucket.
__device__ __forceinline__ void wave_find_bucket(const u32* hist, int need, int* scal, int lane) {
  const u32 c0 = hist[lane * 4 + 0], c1 = hist[lane * 4 + 1];
  const u32 c2 = hist[lane * 4 + 2], c3 = hist[lane * 4 + 3];
  const u32 sum = c0 + c1 + c2 + c3;
  const u32 incl = wave_inclusive_scan(sum, lane);
  const u32 excl = incl - sum;
  const u32 uneed = static_cast<u32>(need);
  const bool mine = excl < uneed && uneed <= incl;
  if (mine) {
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
    scal[0] = b;
    scal[1] = static_cast<int>(run);
    scal[2] = static_cast<int>(cnt);
  }
}

// Exact radix select over M unique packed 48-bit values in LDS: returns the bound B such
// that exactly kk values are <= B (1 <= kk <= M).  8-bit digits, MSB first, early exit as
// soon as a bucket is taken whole.
template <int BLOCK>
__device__ u64 block_select_bound(const u64* list, int M, int kk, u32* hist, int* scal) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  u64 prefix = 0, pmask = 0;
  int need = kk;
  for (int shift = 40; shift >= 0; shift -= 8) {
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
  return prefix | (~pmask & kMask48);
}

// Writes rank r of segment output: index + raw value re-read from the input.  An entry
// outside the segment (only a padding sentinel can be) is written as the pad.
__device__ __forceinline__ void write_rank(const TopkParams& p, int64_t s0, int64_t n, int seg,
                                           int r, u64 P) {
  const u32 idx = static_cast<u32>(P);
  const int64_t o = static_cast<int64_t>(seg) * p.k + r;
  if (r >= p.k) return;
  if (static_cast<int64_t>(idx) < n) {
    p.out_idx[o] = static_cast<int>(idx);
    p.out_vals[o] = p.base[s0 + idx];
  } else {
    p.out_idx[o] = -1;
    p.out_vals[o] = 0xffffu;
  }
}

// Select the kk best of the M packed candidates in LDS (M >= kk) and write them, in order,
// to the segment's output row; ranks kk..k-1 get the pad (index -1, bits 0xFFFF).
template <int BLOCK>
__device__ void finalize_segment(const TopkParams& p, const Smem& sm, int M, int kk, int64_t s0,
                                 int64_t n, int seg) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  if (M < kk) kk = M;  // cannot happen (every candidate list holds >= kk entries); keeps it safe
  for (int r = kk + tid; r < p.k; r += BLOCK) {
    const int64_t o = static_cast<int64_t>(seg) * p.k + r;
    p.out_idx[o] = -1;
    p.out_vals[o] = 0xffffu;
  }
  if (M <= 64) {
    if (wid == 0) {
      u64 x = lane < M ? sm.cand[lane] : ~0ull;
      x = wave_bitonic_sort64(x, lane);
      if (lane < kk) write_rank(p, s0, n, seg, lane, x);
    }
    return;
  }
  const u64* sel = sm.cand;
  if (M > kk) {
    const u64 bound = block_select_bound<BLOCK>(sm.cand, M, kk, sm.hist, sm.scal);
    if (tid == 0) sm.scal[3] = 0;
    __syncthreads();
    for (int i = tid; i < M; i += BLOCK) {
      const u64 P = sm.cand[i];
      if (P <= bound) {
        const int slot = atomicAdd(&sm.scal[3], 1);
        if (slot < p.kpad) sm.sel[slot] = P;
      }
    }
    sel = sm.sel;
  }
  for (int i = tid; i < kk; i += BLOCK) sm.rank[i] = 0;
  __syncthreads();
  // Rank sort: rank(i) = #{j : sel[j] < sel[i]}; the comparisons are split over all threads.
  const int slices = BLOCK / kk > 0 ? BLOCK / kk : 1;
  const int span = (kk + slices - 1) / slices;
  for (int t = tid; t < kk * slices; t += BLOCK) {
    const int i = t % kk;
    const int q = t / kk;
    const int j0 = q * span;
    const int j1 = j0 + span < kk ? j0 + span : kk;
    const u64 P = sel[i];
    int c = 0;
    for (int j = j0; j < j1; ++j) c += sel[j] < P ? 1 : 0;
    if (slices == 1) {
      sm.rank[i] = c;
    } else if (c) {
      atomicAdd(&sm.rank[i], c);
    }
  }
  __syncthreads();
  for (int i = tid; i < kk; i += BLOCK) write_rank(p, s0, n, seg, sm.rank[i], sel[i]);
}

// Epoch-tagged arrival counter: word = epoch << 16 | count.  A word carrying another epoch
// is stale (earlier call, or uninitialised workspace) and counts as zero.  The last
// arriver resets the count to zero, so a replay with the same epoch also works.
__device__ __forceinline__ bool arrive_last(u64* ticket, u64 epoch, int arrivals) {
  u64 old = __hip_atomic_load(ticket, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    const u64 cnt = ((old >> 16) == epoch) ? (old & 0xffffu) : 0u;
    const u64 next = cnt + 1u;
    const bool last = next >= static_cast<u64>(arrivals);
    const u64 word = (epoch << 16) | (last ? 0u : next);
    if (__hip_atomic_compare_exchange_strong(ticket, &old, word, __ATOMIC_ACQ_REL,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
      return last;
    }
  }
}

// ------------------------------------------------------------------------------ the kernel

template <int BLOCK, int VPT>
__global__ void __launch_bounds__(BLOCK) segmented_topk_kernel(TopkParams p) {
  constexpr int NW = BLOCK / 64;
  constexpr int CH = BLOCK * VPT * 8;
  static_assert(CH <= 65536, "chunk positions are packed into 16 bits");
  extern __shared__ __align__(16) unsigned char smem_raw[];
  const Smem sm = carve_smem(smem_raw, p.cand_area, p.kpad);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wid = tid >> 6;
  const int W = p.chunks_per_seg;
  const int seg = static_cast<int>(blockIdx.x) / W;
  const int w = static_cast<int>(blockIdx.x) - seg * W;
  const int k = p.k;

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
  const int64_t a0 = s0 & ~static_cast<int64_t>(7);
  const int64_t span_aligned = s1 - a0;
  const int64_t Ws64 = n > 0 ? (span_aligned + CH - 1) / CH : 0;

  if (n <= 0 || n > p.max_len || Ws64 > W) {
    // Empty segment, or one longer than the declared maximum (broken max_seg_len
    // precondition of the segmented entry point): the whole row is padding.
    if (w == 0) {
      for (int r = tid; r < k; r += BLOCK) {
        const int64_t o = static_cast<int64_t>(seg) * k + r;
        p.out_idx[o] = -1;
        p.out_vals[o] = 0xffffu;
      }
    }
    return;
  }
  const int Ws = static_cast<int>(Ws64);
  if (w >= Ws) return;

  const int kk = n < k ? static_cast<int>(n) : k;
  const int64_t cb = a0 + static_cast<int64_t>(w) * CH;
  const int64_t c0 = s0 > cb ? s0 : cb;
  const int64_t c1 = s1 < cb + CH ? s1 : cb + CH;
  const int nc = static_cast<int>(c1 - c0);
  const int kc = nc < k ? nc : k;
  const int lo = static_cast<int>(c0 - cb);  // valid chunk positions are [lo, hi)
  const int hi = static_cast<int>(c1 - cb);
  const u32 idx_base = static_cast<u32>(cb - s0);  // segment index = idx_base + position

  // ---- 1. load the chunk (one HBM read, 16-byte vectors, coalesced per wave)
  uint4 v[VPT];
  const uint16_t* cptr = p.base + cb;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int pos = (j * BLOCK + tid) * 8;
    if (pos < hi && pos + 8 > lo) {
      v[j] = *reinterpret_cast<const uint4*>(cptr + pos);
      if (pos < lo || pos + 8 > hi) {
        u32 w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (pos + e < lo || pos + e >= hi) w4[e >> 1] |= 0xffffu << ((e & 1) * 16);
        }
        v[j] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
      }
    } else {
      v[j] = make_uint4(kFillWord, kFillWord, kFillWord, kFillWord);
    }
  }

  // ---- 2. thread best (packed int16 max / min over raw bits)
  short2_t mx = {static_cast<short>(-32768), static_cast<short>(-32768)};
  short2_t mn = {32767, 32767};
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const u32 w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const short2_t x = __builtin_bit_cast(short2_t, w4[q]);
      mx = __builtin_elementwise_max(mx, x);
      mn = __builtin_elementwise_min(mn, x);
    }
  }
  const int m1 = mx.x > mx.y ? mx.x : mx.y;
  const int m2 = mn.x < mn.y ? mn.x : mn.y;
  const u32 best_key = desc_key(static_cast<u32>(m1 >= 0 ? m1 : m2) & 0xffffu);

  // ---- 3. threshold T: at least kc real elements of the chunk have key <= T
  const int kw = (kc + NW - 1) / NW;
  if (tid == 0) sm.scal[4] = 0;
  if (kw <= 64) {
    const u32 tw = wave_kth_smallest16(best_key, kw);
    if (lane == 0) sm.wave_t[wid] = tw;
  }
  __syncthreads();
  u32 T = 0xffffu;
  if (kw <= 64) {
    T = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) T = sm.wave_t[i] > T ? sm.wave_t[i] : T;
  }

  // ---- 4. compaction of {key <= T} into the LDS list
  const int cap = p.cap_chunk;
  auto emit = [&](bool hit, u32 b, int pos) {
    const u64 m = ballot(hit);
    if (m) {
      const int leader = __ffsll(static_cast<long long>(m)) - 1;
      int base = 0;
      if (lane == leader) base = atomicAdd(&sm.scal[4], __popcll(m));
      base = static_cast<int>(shfl_u32(static_cast<u32>(base), leader));
      if (hit) {
        const int slot = base + static_cast<int>(mbcnt(m));
        if (slot < cap) sm.cand[slot] = (static_cast<u64>(desc_key(b)) << 32) | (idx_base + static_cast<u32>(pos));
      }
    }
  };

  if (T != 0xffffu) {
    // Integer test on the raw bits equivalent to desc_key(b) <= T for non-NaN b:
    //   T positive (key < 0x7FFF): int16(b) >= int16(raw(T));
    //   T zero or negative:        uint16(b) <= raw(T)  (raw(+-0 class) taken as 0x8000).
    const bool pos_t = T < 0x7fffu;
    const u32 traw = pos_t ? (T ^ 0x7fffu) : (T == 0x7fffu ? 0x8000u : T);
    const int traw_s = static_cast<int>(static_cast<short>(traw));
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const u32 w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const u32 b = (w4[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
        const bool pass = pos_t ? (static_cast<int>(static_cast<short>(b)) >= traw_s) : (b <= traw);
        const bool hit = pass && (b & 0x7fffu) <= 0x7c00u;
        emit(hit, b, (j * BLOCK + tid) * 8 + e);
      }
    }
  } else if (nc <= cap) {
    // No usable threshold (few elements per wave, or NaN-dominated rows): take the chunk.
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const u32 w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int pos = (j * BLOCK + tid) * 8 + e;
        const u32 b = (w4[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
        emit(pos >= lo && pos < hi, b, pos);
      }
    }
  } else if (tid == 0) {
    sm.scal[4] = nc;
  }
  __syncthreads();
  int C = sm.scal[4];

  if (C > cap) {
    // ---- 4b. exact refinement on the registers: radix select over P = key16 << 16 | pos16
    // among in-range elements with key <= T, until at most `cap` values are <= the bound.
    u32 prefix = 0, pmask = 0;
    int need = kc;
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int i = tid; i < 256; i += BLOCK) sm.hist[i] = 0;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        const u32 w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int pos = (j * BLOCK + tid) * 8 + e;
          const u32 key = desc_key((w4[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
          const u32 P = (key << 16) | static_cast<u32>(pos);
          if (pos >= lo && pos < hi && key <= T && (P & pmask) == prefix) {
            atomicAdd(&sm.hist[(P >> shift) & 255u], 1u);
          }
        }
      }
      __syncthreads();
      if (wid == 0) wave_find_bucket(sm.hist, need, sm.scal, lane);
      __syncthreads();
      const int b = sm.scal[0];
      const int before = sm.scal[1];
      const int cnt = sm.scal[2];
      need -= before;
      prefix |= static_cast<u32>(b) << shift;
      pmask |= 0xffu << shift;
      const int count_le = (kc - need) + cnt;
      if (count_le <= cap) break;
    }
    const u32 bound = prefix | ~pmask;
    if (tid == 0) sm.scal[4] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const u32 w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int pos = (j * BLOCK + tid) * 8 + e;
        const u32 b = (w4[e >> 1] >> ((e & 1) * 16)) & 0xffffu;
        const u32 key = desc_key(b);
        const u32 P = (key << 16) | static_cast<u32>(pos);
        emit(pos >= lo && pos < hi && key <= T && P <= bound, b, pos);
      }
    }
    __syncthreads();
    C = sm.scal[4];
  }

  // ---- 5. single-chunk segment: select and write
  if (Ws == 1) {
    finalize_segment<BLOCK>(p, sm, C, kk, s0, n, seg);
    return;
  }

  // ---- 6. multi-chunk segment: publish this chunk's list, last arriver merges
  const u64* src = sm.cand;
  int M = C;
  if (C > p.cap_list) {
    const u64 bound = block_select_bound<BLOCK>(sm.cand, C, kc, sm.hist, sm.scal);
    if (tid == 0) sm.scal[3] = 0;
    __syncthreads();
    for (int i = tid; i < C; i += BLOCK) {
      const u64 P = sm.cand[i];
      if (P <= bound) {
        const int slot = atomicAdd(&sm.scal[3], 1);
        if (slot < p.kpad) sm.sel[slot] = P;
      }
    }
    __syncthreads();
    src = sm.sel;
    M = kc;
  }
  const int64_t list_id = static_cast<int64_t>(seg) * W + w;
  u64* my_list = p.lists + list_id * p.cap_list;
  for (int i = tid; i < M; i += BLOCK) my_list[i] = src[i];
  if (tid == 0) p.list_counts[list_id] = M;
  __threadfence();
  __syncthreads();
  if (tid == 0) sm.scal[5] = arrive_last(p.tickets + seg, p.epoch, Ws) ? 1 : 0;
  __syncthreads();
  if (!sm.scal[5]) return;
  __threadfence();

  int total = 0;
  for (int c = 0; c < Ws; ++c) {
    const int64_t id = static_cast<int64_t>(seg) * W + c;
    int cnt = __hip_atomic_load(p.list_counts + id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    cnt = cnt < 0 ? 0 : (cnt > p.cap_list ? p.cap_list : cnt);
    const u64* lst = p.lists + id * p.cap_list;
    for (int i = tid; i < cnt; i += BLOCK) sm.cand[total + i] = lst[i];
    total += cnt;
  }
  __syncthreads();
  finalize_segment<BLOCK>(p, sm, total, kk, s0, n, seg);
}

template <int BLOCK, int VPT>
int launch_shape(const Plan& plan, const TopkParams& params, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(params.seg_num) * plan.W));
  hipLaunchKernelGGL((segmented_topk_kernel<BLOCK, VPT>), grid, dim3(BLOCK),
                     static_cast<unsigned>(plan.lds_bytes), stream, params);
  return static_cast<int>(hipGetLastError());
}

}  // namespace

int launch_segmented_topk(const Plan& plan, const TopkParams& params, void* stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int b = plan.shape.block;
  const int vpt = plan.shape.vpt;
  if (b == 256 && vpt == 2) return launch_shape<256, 2>(plan, params, s);
  if (b == 256 && vpt == 4) return launch_shape<256, 4>(plan, params, s);
  if (b == 256 && vpt == 8) return launch_shape<256, 8>(plan, params, s);
  if (b == 512 && vpt == 2) return launch_shape<512, 2>(plan, params, s);
  if (b == 512 && vpt == 4) return launch_shape<512, 4>(plan, params, s);
  if (b == 512 && vpt == 8) return launch_shape<512, 8>(plan, params, s);
  if (b == 1024 && vpt == 2) return launch_shape<1024, 2>(plan, params, s);
  if (b == 1024 && vpt == 4) return launch_shape<1024, 4>(plan, params, s);
  if (b == 1024 && vpt == 8) return launch_shape<1024, 8>(plan, params, s);
  return static_cast<int>(hipErrorInvalidValue);
}

}  // namespace radix_topk_amd
