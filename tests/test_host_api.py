"""Host-side checks of the C ABI that need no GPU: the library loads, exports every symbol
include/batch_topk.h declares, validates arguments before any HIP call (reference
src/batch_topk.cu:13-33 and test/test_batch_topk.cu:1168-1174,1311-1373), and sizes the
workspace from the shape alone (src/batch_topk.cu:35-40)."""

import os
import re
import subprocess

import pytest

import batch_topk_amd as bt

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INVALID = bt.HIP_ERROR_INVALID_VALUE
# Dummy, never-dereferenced device addresses: every call below is rejected before use.
P_IN, P_VAL, P_IDX, P_WS, P_OFF = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000


def declared_symbols():
    with open(os.path.join(ROOT, "include", "batch_topk.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|void)\s+(radix_topk_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = bt.load_library()
    decl = declared_symbols()
    assert decl == sorted(bt.EXPORTED_SYMBOLS)
    for name in decl:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", bt.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(line.split()[-1] for line in out.splitlines() if " T " in line)
    assert set(decl) <= exported


def test_phase_trace_hooks_only_in_the_measurement_build():
    # The per-phase clock stamps are compiled into libbatch_topk_amd_trace.so (loaded by
    # batch_topk_amd.profiling only); the engine library has no trace entry point.
    from batch_topk_amd import build

    def defined(path):
        out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                             check=True).stdout
        return set(line.split()[-1] for line in out.splitlines() if " T " in line)

    if not os.path.exists(build.TRACE_LIB_PATH):
        pytest.skip("measurement libraries not built")
    trace = defined(build.TRACE_LIB_PATH)
    assert {"radix_topk_trace_fetch", "radix_topk_trace_clear"} <= trace
    assert set(declared_symbols()) <= trace
    assert not any("trace" in name for name in defined(bt.LIB_PATH))


def test_cpp_dropin_header_forwards_to_c_abi(tmp_path):
    # The C++ drop-in (include/batch_topk.hpp) compiles against HIP headers and adds no symbols.
    src = tmp_path / "use.cpp"
    src.write_text('#include "batch_topk.hpp"\n'
                   'size_t f(int a, int b, int c) { return radix_topk::batch_topk_half_workspace_size(a, b, c); }\n'
                   'hipError_t g(const __half* x, __half* v, int* i, void* w, size_t n, hipStream_t s) {\n'
                   '  return radix_topk::batch_topk_half(x, 1, 8, 3, v, i, w, n, s); }\n'
                   'hipError_t h(const __hip_bfloat16* x, __hip_bfloat16* v, int* i, void* w, size_t n,\n'
                   '             hipStream_t s) { return radix_topk::batch_topk_bf16(x, 1, 8, 3, v, i, w, n, s); }\n')
    res = subprocess.run(["g++", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROOT, "include"),
                          "-I", "/opt/rocm/include", "-c", str(src), "-o", str(tmp_path / "use.o")],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stderr


def test_workspace_size_contract():
    # invalid shapes -> 0 (test/test_batch_topk.cu:1168-1174 keeps (0,10000,50) and (1,10,11))
    assert bt.batch_topk_half_workspace_size(0, 10000, 50) == 0
    assert bt.batch_topk_half_workspace_size(1, 10, 11) == 0
    assert bt.batch_topk_half_workspace_size(1, 10000, 0) == 0
    assert bt.batch_topk_half_workspace_size(1, 0, 1) == 0
    assert bt.batch_topk_half_workspace_size(1, 2000, bt.MAX_K + 1) == 0
    # lifted envelope: the reference's seg_len <= 10000 and k <= 128 limits are gone
    assert bt.batch_topk_half_workspace_size(1, 10001, 50) > 1
    assert bt.batch_topk_half_workspace_size(1, 10000, 129) > 1
    assert bt.batch_topk_half_workspace_size(128, 128256, 50) > 1
    assert bt.batch_topk_half_workspace_size(256, 32000, 256) > 1
    # segments up to 2^31 - 1 elements at every k (the long-segment path beyond one
    # co-resident grid of single-chunk workgroups)
    for shape in ((1, 50_000_000, 1), (1, 50_000_000, 1024), (4, 20_000_000, 64), (300, 200_000, 1024),
                  (1, 2**31 - 1, 1024), (2, 2**30, 1), (5000, 400_000, 700)):
        assert bt.batch_topk_half_workspace_size(*shape) > 1, shape
    assert bt.batch_topk_half_segmented_workspace_size(218, 131072, 1024) > 1
    assert bt.batch_topk_half_segmented_workspace_size(3, 2**31 - 1, 64) > 1
    # > 1 so that "workspace_bytes - 1" is a meaningful short workspace (test:1311-1314)
    ws = bt.batch_topk_half_workspace_size(1, 10000, 50)
    assert ws > 1
    # far below the legacy per-element Candidate storage (test:270-280)
    assert bt.batch_topk_half_workspace_size(128, 10000, 50) < 128 * 10000 * 12
    # shape-only: repeated queries agree
    assert ws == bt.batch_topk_half_workspace_size(1, 10000, 50)
    # segmented variant
    assert bt.batch_topk_half_segmented_workspace_size(512, 65536, 64) > 1
    assert bt.batch_topk_half_segmented_workspace_size(0, 65536, 64) == 0
    assert bt.batch_topk_half_segmented_workspace_size(4, -1, 64) == 0
    assert bt.batch_topk_half_segmented_workspace_size(4, 100, 0) == 0


def test_noalloc_entry_point_rejects_before_any_hip_call():
    # invalid arguments as the plain entry point (1), and a shape whose workspace exceeds the
    # static per-GPU array (2 = hipErrorOutOfMemory), all before any HIP call
    call = bt.batch_topk_half_noalloc
    assert call(0, 1, 10000, 50, P_VAL, P_IDX) == INVALID
    assert call(P_IN, 1, 10000, 50, 0, P_IDX) == INVALID
    assert call(P_IN, 1, 10000, 50, P_VAL, 0) == INVALID
    assert call(P_IN, 1, 10, 11, P_VAL, P_IDX) == INVALID
    assert call(P_IN, 0, 10000, 50, P_VAL, P_IDX) == INVALID
    assert call(P_IN, 1, 10000, bt.MAX_K + 1, P_VAL, P_IDX) == INVALID
    big = (128, 16_000_000, 64)
    assert bt.batch_topk_half_workspace_size(*big) > bt.NOALLOC_SCRATCH_BYTES
    assert call(P_IN, *big, P_VAL, P_IDX) == bt.HIP_ERROR_OUT_OF_MEMORY
    # the workloads of the benchmark fit it
    for shape in ((16, 4096, 50), (128, 128256, 50), (256, 32000, 256), (1, 1 << 24, 1024),
                  (1, 50_000_000, 1024)):
        assert 0 < bt.batch_topk_half_workspace_size(*shape) <= bt.NOALLOC_SCRATCH_BYTES, shape


def test_validation_rejects_before_any_hip_call():
    ws = bt.batch_topk_half_workspace_size(1, 10000, 50)
    call = bt.batch_topk_half
    # null pointers (test/test_batch_topk.cu:1340-1373)
    assert call(0, 1, 10000, 50, P_VAL, P_IDX, P_WS, ws) == INVALID
    assert call(P_IN, 1, 10000, 50, 0, P_IDX, P_WS, ws) == INVALID
    assert call(P_IN, 1, 10000, 50, P_VAL, 0, P_WS, ws) == INVALID
    assert call(P_IN, 1, 10000, 50, P_VAL, P_IDX, 0, ws) == INVALID
    # k > seg_len, bad sizes
    assert call(P_IN, 1, 10, 11, P_VAL, P_IDX, P_WS, 1 << 20) == INVALID
    assert call(P_IN, 0, 10, 1, P_VAL, P_IDX, P_WS, 1 << 20) == INVALID
    assert call(P_IN, 1, 0, 1, P_VAL, P_IDX, P_WS, 1 << 20) == INVALID
    assert call(P_IN, 1, 10, 0, P_VAL, P_IDX, P_WS, 1 << 20) == INVALID
    assert call(P_IN, 1, 5000, bt.MAX_K + 1, P_VAL, P_IDX, P_WS, 1 << 30) == INVALID
    # short workspace (test/test_batch_topk.cu:1375-1385)
    assert call(P_IN, 1, 10000, 50, P_VAL, P_IDX, P_WS, ws - 1) == INVALID
    # misaligned element pointers
    assert call(P_IN + 1, 1, 10000, 50, P_VAL, P_IDX, P_WS, ws) == INVALID
    assert call(P_IN, 1, 10000, 50, P_VAL + 1, P_IDX, P_WS, ws) == INVALID
    assert call(P_IN, 1, 10000, 50, P_VAL, P_IDX + 2, P_WS, ws) == INVALID


def test_segmented_validation_rejects_before_any_hip_call():
    ws = bt.batch_topk_half_segmented_workspace_size(4, 1000, 64)
    call = bt.batch_topk_half_segmented
    assert call(0, P_OFF, 4, 1000, 64, P_VAL, P_IDX, P_WS, ws) == INVALID
    assert call(P_IN, 0, 4, 1000, 64, P_VAL, P_IDX, P_WS, ws) == INVALID
    assert call(P_IN, P_OFF, 0, 1000, 64, P_VAL, P_IDX, P_WS, ws) == INVALID
    assert call(P_IN, P_OFF, 4, -1, 64, P_VAL, P_IDX, P_WS, ws) == INVALID
    assert call(P_IN, P_OFF, 4, 1000, 0, P_VAL, P_IDX, P_WS, ws) == INVALID
    assert call(P_IN, P_OFF, 4, 1000, 64, P_VAL, P_IDX, P_WS, ws - 1) == INVALID
    assert call(P_IN, P_OFF + 2, 4, 1000, 64, P_VAL, P_IDX, P_WS, ws) == INVALID


def test_torch_helpers_fail_loudly_without_gpu():
    torch = pytest.importorskip("torch")
    x = torch.zeros((2, 8), dtype=torch.float16)
    with pytest.raises(ValueError):
        bt.topk(x, 3)   # CPU tensor: there is no CPU fallback


def test_kernel_resources_keep_occupancy_without_spills():
    # Every instantiation must run at least 4 waves per SIMD (one 1024-thread or two
    # 512-thread workgroups per CU) with no scratch spills: the kernels are latency-bound,
    # and a lost workgroup slot or a spill shows up directly in the per-call time.
    from batch_topk_amd.build import resource_usage

    usage = resource_usage()
    kernels = {k: v for k, v in usage.items() if "segmented_topk_kernel" in k}
    # 12 workgroup shapes + the two cooperative ones (8 and 16 vectors), plus the 12 shapes again
    # with the short-chunk threshold, each for 16-bit and for 32-bit elements
    assert len(kernels) == 52, sorted(kernels)
    assert sum("Elem32" in k for k in kernels) == 26, sorted(kernels)
    # and the long-segment kernel for 16-bit and 32-bit elements
    long_kernels = {k: v for k, v in usage.items() if "long_segment_kernel" in k}
    assert len(long_kernels) == 2, sorted(long_kernels)
    kernels.update(long_kernels)
    for name, r in kernels.items():
        assert r["ScratchSize [bytes/lane]"] == 0, (name, r)
        assert r["Occupancy [waves/SIMD]"] >= 4, (name, r)


def test_sample_validation_rejects_before_any_hip_call():
    ws = bt.sample_half_workspace_size(2, 1000, 50)
    assert ws == bt.batch_topk_half_workspace_size(2, 1000, 50) > 1
    assert bt.sample_bf16_workspace_size(2, 1000, 50) == ws
    P_U, P_S, P_PR = 0x60000, 0x70000, 0x80000
    for fn in (bt.sample_half, bt.sample_bf16):
        ok = dict(d_logits=P_IN, seg_num=2, seg_len=1000, k=50, temperature=1.0, d_uniforms=P_U,
                  d_topk_values=P_VAL, d_topk_indices=P_IDX, d_probs=P_PR, d_samples=P_S,
                  d_workspace=P_WS, workspace_bytes=ws)
        for bad in (dict(temperature=0.0), dict(temperature=-1.0), dict(temperature=float("nan")),
                    dict(temperature=float("inf")), dict(temperature=1e-45),
                    dict(d_uniforms=0), dict(d_samples=0), dict(d_logits=0), dict(d_topk_values=0),
                    dict(d_topk_indices=0), dict(d_workspace=0), dict(k=0), dict(k=1001),
                    dict(seg_num=0), dict(workspace_bytes=ws - 1)):
            assert fn(**dict(ok, **bad)) == INVALID, (fn.__name__, bad)


def test_f32_entry_points_validate_and_size():
    # fp32 rows are planned with four elements per 16-byte load: their own workspace sizes
    assert bt.batch_topk_f32_workspace_size(128, 128256, 50) > 1
    assert bt.batch_topk_f32_workspace_size(1, 10, 11) == 0
    assert bt.batch_topk_f32_workspace_size(0, 10, 1) == 0
    assert bt.batch_topk_f32_segmented_workspace_size(4, 1000, 64) > 1
    assert bt.batch_topk_ex_workspace_size(bt.FORMAT_F32, False, 128, 128256, 50) == \
        bt.batch_topk_f32_workspace_size(128, 128256, 50)
    assert bt.batch_topk_ex_workspace_size(bt.FORMAT_F32, True, 4, 1000, 64) == \
        bt.batch_topk_f32_segmented_workspace_size(4, 1000, 64)
    # 2^24 floats with k = 1024 take 256 cooperative chunks when 16-byte aligned (a misaligned
    # pointer is refused at launch); longer rows, or more of them, take the long-segment path
    assert bt.batch_topk_f32_workspace_size(1, 1 << 24, 1024) > 1
    assert bt.batch_topk_f32_workspace_size(2, 1 << 24, 1024) > 1
    assert bt.batch_topk_f32_workspace_size(1, (1 << 24) + 1, 1024) > 1
    assert bt.batch_topk_f32_workspace_size(1, 2**31 - 1, 1024) > 1
    ws = bt.batch_topk_f32_workspace_size(1, 10000, 50)
    call = bt.batch_topk_f32
    assert call(0, 1, 10000, 50, P_VAL, P_IDX, P_WS, ws) == INVALID
    assert call(P_IN, 1, 10000, 50, 0, P_IDX, P_WS, ws) == INVALID
    assert call(P_IN, 1, 10, 11, P_VAL, P_IDX, P_WS, 1 << 20) == INVALID
    assert call(P_IN, 1, 10000, 50, P_VAL, P_IDX, P_WS, ws - 1) == INVALID
    assert call(P_IN + 2, 1, 10000, 50, P_VAL, P_IDX, P_WS, ws) == INVALID   # floats: 4-byte aligned
    assert call(P_IN, 1, 10000, 50, P_VAL + 2, P_IDX, P_WS, ws) == INVALID
    seg = bt.batch_topk_f32_segmented
    wss = bt.batch_topk_f32_segmented_workspace_size(4, 1000, 64)
    assert seg(P_IN, 0, 4, 1000, 64, P_VAL, P_IDX, P_WS, wss) == INVALID
    assert seg(P_IN + 2, P_OFF, 4, 1000, 64, P_VAL, P_IDX, P_WS, wss) == INVALID


def test_ex_workspace_matches_the_plain_entry_points():
    for fmt in (bt.FORMAT_F16, bt.FORMAT_BF16):
        for shape in ((1, 10000, 50), (128, 128256, 50), (3, 250000, 512), (1, 16777216, 1024)):
            assert bt.batch_topk_ex_workspace_size(fmt, False, *shape) == bt.batch_topk_half_workspace_size(*shape)
            assert bt.batch_topk_ex_workspace_size(fmt, True, *shape) == \
                bt.batch_topk_half_segmented_workspace_size(*shape)
    assert bt.batch_topk_ex_workspace_size(3, False, 1, 10000, 50) == 0   # unknown format
    assert bt.batch_topk_ex_workspace_size(bt.FORMAT_F16, False, 1, 10, 11) == 0
    assert bt.batch_topk_ex_workspace_size(bt.FORMAT_F16, True, 1, 10, 11) > 1  # short segments pad


def test_ex_validation_rejects_before_any_hip_call():
    ws = bt.batch_topk_ex_workspace_size(bt.FORMAT_F16, True, 4, 1000, 64)
    ok = dict(d_input=P_IN, fmt=bt.FORMAT_F16, d_offsets=P_OFF, seg_num=4, seg_len=1000, k=64, flags=0,
              d_output_values=P_VAL, d_output_indices=P_IDX, d_workspace=P_WS, workspace_bytes=ws)
    for bad in (dict(fmt=3), dict(fmt=-1), dict(flags=4), dict(flags=-1),
                dict(d_output_values=0), dict(d_output_values=0, flags=bt.UNSORTED),
                dict(d_input=0), dict(d_output_indices=0), dict(d_workspace=0),
                dict(seg_num=0), dict(seg_len=-1), dict(k=0), dict(k=bt.MAX_K + 1),
                dict(workspace_bytes=ws - 1), dict(d_input=P_IN + 1), dict(d_output_indices=P_IDX + 2),
                dict(d_offsets=0, seg_len=10, k=11),   # fixed length: k > seg_len
                dict(d_offsets=0, seg_len=0)):
        assert bt.batch_topk_ex(**dict(ok, **bad)) == INVALID, bad
