// Measurement reference, not part of the top-k engine: the cheapest possible single pass over
// a batch of fp16 rows, to measure the launch and HBM floor a one-launch top-k of the same
// shape cannot beat on this GPU.  Every element is read once with the same nontemporal
// 16-byte loads as the top-k kernel (all issued before any is used), reduced to one word per
// wave with a VALU max and a lane read, and one word per wave is stored.  Built into
// libread_floor.so; batch_topk_amd/profiling.py ("floor") times it back-to-back.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

// Workgroup b reads chunk (b % W) of row (b / W); chunks are `chunk` elements (a multiple
// of 8), the last one of a row is shorter.  Lanes whose vector lies past the chunk re-read
// the chunk's first vector, so every load stays inside the row.
template <int BLOCK, int VPT>
__global__ void __launch_bounds__(BLOCK) read_floor_kernel(const uint16_t* in, int row_len, int W,
                                                           int chunk, unsigned* out) {
  const int r = blockIdx.x / W;
  const int c = blockIdx.x - r * W;
  const unsigned char* base =
      reinterpret_cast<const unsigned char*>(in + static_cast<size_t>(r) * row_len + static_cast<size_t>(c) * chunk);
  int lim = row_len - c * chunk;
  if (lim > chunk) lim = chunk;
  u32x4_t v[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    int pos = (j * BLOCK + static_cast<int>(threadIdx.x)) * 8;
    if (pos + 8 > lim) pos = 0;
    v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(base + pos * 2));
  }
  unsigned m = 0;
#pragma unroll
  for (int j = 0; j < VPT; ++j) m = max(m, max(max(v[j].x, v[j].y), max(v[j].z, v[j].w)));
  m = max(m, static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(m), 63)));
  if ((threadIdx.x & 63) == 0) out[blockIdx.x * (BLOCK / 64) + (threadIdx.x >> 6)] = m;
}

// The same read with one 1024-thread workgroup per row and 16 vectors per thread, stamping
// per wave (lane 0, shader clock) its start, the moment its 16 loads are issued and the moment
// all its data is in (after a dependent reduction), into stamps[(row * 16 + wave) * 3 + i].
// `barrier_first` adds a workgroup barrier before the loads.  Shows in what order a CU serves
// the loads of its waves.
__device__ __forceinline__ unsigned long long shader_clock() {
  unsigned long long t;
  asm volatile("s_memtime %0\n s_waitcnt lgkmcnt(0)" : "=s"(t)::"memory");
  return t;
}
__global__ void __launch_bounds__(1024) arrival_kernel(const uint16_t* in, int row_len, int barrier_first,
                                                       unsigned* out, unsigned long long* stamps) {
  const unsigned long long c0 = shader_clock();
  const unsigned char* base = reinterpret_cast<const unsigned char*>(in + static_cast<size_t>(blockIdx.x) * row_len);
  if (barrier_first) __syncthreads();
  u32x4_t v[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    int pos = (j * 1024 + static_cast<int>(threadIdx.x)) * 8;
    if (pos + 8 > row_len) pos = 0;
    v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(base + pos * 2));
  }
  const unsigned long long c1 = shader_clock();
  unsigned m = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) m = max(m, max(max(v[j].x, v[j].y), max(v[j].z, v[j].w)));
  m = max(m, static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(m), 63)));
  const unsigned long long c2 = shader_clock();
  if ((threadIdx.x & 63) == 0) {
    const int wv = static_cast<int>(blockIdx.x) * 16 + static_cast<int>(threadIdx.x >> 6);
    out[wv] = m;
    stamps[wv * 3 + 0] = c0;
    stamps[wv * 3 + 1] = c1;
    stamps[wv * 3 + 2] = c2;
  }
}

// A kernel that does nothing: the launch cost alone.
__global__ void __launch_bounds__(1024) empty_kernel(unsigned* out) {
  if (threadIdx.x == 0x7fffffff) out[0] = 1;
}

template <int BLOCK, int VPT>
int launch(const uint16_t* in, int rows, int row_len, int W, unsigned* out, hipStream_t s) {
  const int chunk = ((row_len + W - 1) / W + 7) / 8 * 8;
  if (static_cast<long>(BLOCK) * VPT * 8 < chunk) return static_cast<int>(hipErrorInvalidValue);
  hipLaunchKernelGGL((read_floor_kernel<BLOCK, VPT>), dim3(static_cast<unsigned>(rows * W)), dim3(BLOCK), 0,
                     s, in, row_len, W, chunk, out);
  return static_cast<int>(hipGetLastError());
}

}  // namespace

// One back-to-back launch per entry of `inputs` (device pointers, `calls` of them).  `out`
// needs rows * W * block / 64 words.  Shapes: (block, vpt, W) = (1024, 16, 1), (512, 32, 1),
// (512, 16, 2), (256, 16, 4), (1024, 8, 2).
extern "C" int read_floor_run(const uint16_t* const* inputs, int calls, int rows, int row_len,
                              int block, int vpt, int W, unsigned* out, void* stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  for (int i = 0; i < calls; ++i) {
    int rc;
    if (block == 1024 && vpt == 16) rc = launch<1024, 16>(inputs[i], rows, row_len, W, out, s);
    else if (block == 512 && vpt == 32) rc = launch<512, 32>(inputs[i], rows, row_len, W, out, s);
    else if (block == 512 && vpt == 16) rc = launch<512, 16>(inputs[i], rows, row_len, W, out, s);
    else if (block == 256 && vpt == 16) rc = launch<256, 16>(inputs[i], rows, row_len, W, out, s);
    else if (block == 1024 && vpt == 8) rc = launch<1024, 8>(inputs[i], rows, row_len, W, out, s);
    else rc = static_cast<int>(hipErrorInvalidValue);
    if (rc != 0) return rc;
  }
  return 0;
}

// `calls` back-to-back launches of the arrival kernel over inputs[i] (rows of row_len fp16, at
// most 131,072); the stamps of the last launch stay in `stamps` (rows * 16 * 3 words), `out`
// needs rows * 16 words.
extern "C" int read_floor_arrival_run(const uint16_t* const* inputs, int calls, int rows, int row_len,
                                      int barrier_first, unsigned* out, unsigned long long* stamps, void* stream) {
  if (row_len <= 0 || row_len > 1024 * 16 * 8) return static_cast<int>(hipErrorInvalidValue);
  for (int i = 0; i < calls; ++i) {
    hipLaunchKernelGGL(arrival_kernel, dim3(static_cast<unsigned>(rows)), dim3(1024), 0,
                       static_cast<hipStream_t>(stream), inputs[i], row_len, barrier_first, out, stamps);
  }
  return static_cast<int>(hipGetLastError());
}

// `calls` back-to-back launches of an empty kernel with `rows` workgroups of 1024 threads.
extern "C" int read_floor_empty_run(int calls, int rows, unsigned* out, void* stream) {
  for (int i = 0; i < calls; ++i) {
    hipLaunchKernelGGL(empty_kernel, dim3(static_cast<unsigned>(rows)), dim3(1024), 0,
                       static_cast<hipStream_t>(stream), out);
  }
  return static_cast<int>(hipGetLastError());
}
