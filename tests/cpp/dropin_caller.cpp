// A C++ caller of the reference's host API, compiled against this repository's drop-in header
// (include/batch_topk.hpp) and linked against libbatch_topk_amd.so: the calls are spelled as a
// caller of radix_topk::batch_topk_half (reference include/batch_topk.cuh:10-21) spells them,
// with HIP types.  Driven by tests/test_cpp_dropin_gpu.py.
//
//   dropin_caller CASES_FILE
//
// First the argument checks of the reference's API sequence (test/test_batch_topk.cu:1302-1385:
// NULL pointers, k > seg_len, a workspace one byte short, then a successful call on an all-zero
// row), then every case of CASES_FILE, each with its own workspace (poisoned with 0xA5 bytes when
// the case asks for it).  CASES_FILE: the case count, then per case a line
// "name seg_num seg_len k poison" and a line of seg_num * seg_len fp16 bit patterns (decimal).
// Output: "api ok", then per case "case NAME", a line of indices and a line of value bits.
// Exit status 0 when every step succeeded.

#include <cstdint>
#include <cstdio>
#include <fstream>
#include <string>
#include <vector>

#include "batch_topk.hpp"

namespace {

int fail(const char* what) {
  std::fprintf(stderr, "dropin_caller: %s\n", what);
  return 1;
}

struct DeviceBuffers {
  __half* input = nullptr;
  __half* values = nullptr;
  int* indices = nullptr;
  void* workspace = nullptr;
  ~DeviceBuffers() {
    (void)hipFree(workspace);
    (void)hipFree(indices);
    (void)hipFree(values);
    (void)hipFree(input);
  }
  bool allocate(size_t elements, size_t outputs, size_t ws_bytes) {
    return hipMalloc(reinterpret_cast<void**>(&input), sizeof(__half) * elements) == hipSuccess &&
           hipMalloc(reinterpret_cast<void**>(&values), sizeof(__half) * outputs) == hipSuccess &&
           hipMalloc(reinterpret_cast<void**>(&indices), sizeof(int) * outputs) == hipSuccess &&
           hipMalloc(&workspace, ws_bytes) == hipSuccess;
  }
};

// The reference's argument checks, then one successful call on a zero row of 10,000 (k = 50).
int api_sequence() {
  const int seg_num = 1, seg_len = 10000, k = 50;
  const size_t ws = radix_topk::batch_topk_half_workspace_size(seg_num, seg_len, k);
  if (ws <= 1) return fail("workspace size of a valid shape must exceed one byte");
  if (radix_topk::batch_topk_half_workspace_size(1, 10, 11) != 0) return fail("k > seg_len must size to 0");
  DeviceBuffers b;
  if (!b.allocate(seg_len, k, ws)) return fail("hipMalloc");
  if (hipMemset(b.input, 0, sizeof(__half) * seg_len) != hipSuccess) return fail("hipMemset");
  const hipError_t bad = hipErrorInvalidValue;
  if (radix_topk::batch_topk_half(nullptr, seg_num, seg_len, k, b.values, b.indices, b.workspace, ws, 0) != bad ||
      radix_topk::batch_topk_half(b.input, seg_num, seg_len, k, nullptr, b.indices, b.workspace, ws, 0) != bad ||
      radix_topk::batch_topk_half(b.input, seg_num, seg_len, k, b.values, nullptr, b.workspace, ws, 0) != bad ||
      radix_topk::batch_topk_half(b.input, seg_num, seg_len, k, b.values, b.indices, nullptr, ws, 0) != bad ||
      radix_topk::batch_topk_half(b.input, 1, 10, 11, b.values, b.indices, b.workspace,
                                  radix_topk::batch_topk_half_workspace_size(1, 10, 11), 0) != bad) {
    return fail("invalid arguments must be rejected with hipErrorInvalidValue");
  }
  if (radix_topk::batch_topk_half(b.input, seg_num, seg_len, k, b.values, b.indices, b.workspace, ws - 1, 0) != bad) {
    return fail("a workspace one byte short must be rejected");
  }
  if (radix_topk::batch_topk_half(b.input, seg_num, seg_len, k, b.values, b.indices, b.workspace, ws, 0) != hipSuccess ||
      hipDeviceSynchronize() != hipSuccess) {
    return fail("the valid call must succeed");
  }
  std::vector<int> idx(k);
  if (hipMemcpy(idx.data(), b.indices, sizeof(int) * k, hipMemcpyDeviceToHost) != hipSuccess) return fail("copy");
  for (int r = 0; r < k; ++r) {
    if (idx[r] != r) return fail("a zero row must give indices 0..k-1 (ties by ascending index)");
  }
  std::printf("api ok\n");
  return 0;
}

int run_case(const std::string& name, int seg_num, int seg_len, int k, bool poison,
             const std::vector<uint16_t>& bits) {
  const size_t ws = radix_topk::batch_topk_half_workspace_size(seg_num, seg_len, k);
  if (ws == 0) return fail("unsupported case shape");
  const size_t outputs = static_cast<size_t>(seg_num) * k;
  DeviceBuffers b;
  if (!b.allocate(bits.size(), outputs, ws)) return fail("hipMalloc");
  if (hipMemcpy(b.input, bits.data(), sizeof(uint16_t) * bits.size(), hipMemcpyHostToDevice) != hipSuccess ||
      hipMemset(b.workspace, poison ? 0xA5 : 0, ws) != hipSuccess) {
    return fail("input copy");
  }
  hipStream_t stream = nullptr;
  if (hipStreamCreate(&stream) != hipSuccess) return fail("hipStreamCreate");
  const hipError_t rc =
      radix_topk::batch_topk_half(b.input, seg_num, seg_len, k, b.values, b.indices, b.workspace, ws, stream);
  const hipError_t sync = hipStreamSynchronize(stream);
  (void)hipStreamDestroy(stream);
  if (rc != hipSuccess || sync != hipSuccess) return fail("batch_topk_half failed");
  std::vector<int> idx(outputs);
  std::vector<uint16_t> vals(outputs);
  if (hipMemcpy(idx.data(), b.indices, sizeof(int) * outputs, hipMemcpyDeviceToHost) != hipSuccess ||
      hipMemcpy(vals.data(), b.values, sizeof(uint16_t) * outputs, hipMemcpyDeviceToHost) != hipSuccess) {
    return fail("output copy");
  }
  std::printf("case %s\n", name.c_str());
  for (size_t i = 0; i < outputs; ++i) std::printf("%d%c", idx[i], i + 1 == outputs ? '\n' : ' ');
  for (size_t i = 0; i < outputs; ++i) std::printf("%u%c", vals[i], i + 1 == outputs ? '\n' : ' ');
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) return fail("usage: dropin_caller CASES_FILE");
  if (api_sequence() != 0) return 1;
  std::ifstream in(argv[1]);
  int cases = 0;
  if (!(in >> cases)) return fail("cannot read the case count");
  for (int c = 0; c < cases; ++c) {
    std::string name;
    int seg_num = 0, seg_len = 0, k = 0, poison = 0;
    if (!(in >> name >> seg_num >> seg_len >> k >> poison) || seg_num <= 0 || seg_len <= 0) {
      return fail("malformed case header");
    }
    std::vector<uint16_t> bits(static_cast<size_t>(seg_num) * seg_len);
    for (auto& v : bits) {
      unsigned x = 0;
      if (!(in >> x) || x > 0xFFFFu) return fail("malformed case data");
      v = static_cast<uint16_t>(x);
    }
    if (run_case(name, seg_num, seg_len, k, poison != 0, bits) != 0) return 1;
  }
  return 0;
}
