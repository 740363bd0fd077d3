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

// `calls` back-to-back launches of an empty kernel with `rows` workgroups of 1024 threads.
extern "C" int read_floor_empty_run(int calls, int rows, unsigned* out, void* stream) {
  for (int i = 0; i < calls; ++i) {
    hipLaunchKernelGGL(empty_kernel, dim3(static_cast<unsigned>(rows)), dim3(1024), 0,
                       static_cast<hipStream_t>(stream), out);
  }
  return static_cast<int>(hipGetLastError());
}
