"""GPU parity of the one-workgroup-per-chunk kernels on periodic rows.

Those kernels give thread t, as its vector j, slot (t + 64 j) mod BLOCK of the j-th block of
BLOCK vectors.  The rotation matters on data whose period divides the block stride: the
reference bench's fill (bench/bench_batch_topk.cu:9-15) repeats every 2,048 elements, the
stride of 256 threads x 8 fp16 elements.  These cases put such rows through every workgroup
shape of at most 8 vectors per thread: misaligned starts (vector 0 and the tail vectors
masked), two-chunk rows, segmented batches, bfloat16 and fp32, and k from 1 to 256."""

import numpy as np
import pytest

import batch_topk_amd as bt
from oracle import oracle as O
from tests.gpu_util import announce, assert_same, run_fixed, run_segmented

pytestmark = pytest.mark.gpu

THREADS = 8


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    bt.load_library()


def _periodic(n, period, fmt="f16"):
    """(i * 17 + 13) mod period, centred and scaled as the reference bench fills its rows."""
    i = np.arange(n, dtype=np.int64)
    x = (((i * 17 + 13) % period) - period // 2).astype(np.float32) / np.float32(16.0)
    if fmt == "bf16":
        import torch

        return torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    if fmt == "f32":
        return x.view(np.uint32).copy()
    return x.astype(np.float16).view(np.uint16)


# (seg_num, seg_len, k, period, elem_offset); the plan's workgroup shape in the comment
@pytest.mark.parametrize("seg_num,seg_len,k,period,elem_offset", [
    (1500, 16000, 50, 2048, 5),    # 256 x 8, misaligned starts
    (1500, 10000, 50, 2048, 0),    # 256 x 8, the reference matrix's row length
    (700, 10000, 1, 2048, 3),      # 256 x 8, k = 1
    (600, 16384, 256, 2048, 0),    # 1024 x 2, a tail chunk for the worst-case span
    (300, 60000, 64, 2048, 3),     # 1024 x 8, one chunk a row
    (128, 10000, 128, 2048, 0),    # 1024 x 2
    (2000, 3000, 16, 1024, 1),     # 256 x 2
    (1000, 8192, 100, 4096, 7),    # 512 x 2 and tail chunks; the period is its block stride
])
def test_periodic_rows(seg_num, seg_len, k, period, elem_offset):
    bits = _periodic(seg_num * seg_len, period).reshape(seg_num, seg_len)
    exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS)
    announce(f"periodic {seg_num}x{seg_len} k={k} period={period} offset={elem_offset}")
    got = run_fixed(bits, k, poison=0xA5, elem_offset=elem_offset)
    assert_same(got, exp, f"periodic {seg_num}x{seg_len} k={k}")


def test_periodic_segmented():
    rng = np.random.default_rng(2048)
    lengths = rng.integers(1, 16385, size=2000).astype(np.int64)
    lengths[:3] = [16384, 0, 2048]
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    bits = _periodic(int(offsets[-1]), 2048)
    exp = O.batch_topk_half(bits, 50, offsets=offsets.astype(np.int64), threads=THREADS)
    announce("periodic segmented 2000 x U[1,16384] k=50")
    got = run_segmented(bits, offsets, 50, 16384, elem_offset=3, poison=0x5A)
    assert_same(got, exp, "periodic segmented")


def test_periodic_bf16():
    bits = _periodic(1500 * 12000, 2048, fmt="bf16").reshape(1500, 12000)
    exp = O.batch_topk_half(bits, 50, seg_len=12000, threads=THREADS, fmt="bf16")
    announce("periodic bf16 1500x12000 k=50")
    assert_same(run_fixed(bits, 50, poison=0xA5, fmt="bf16", elem_offset=2), exp, "periodic bf16")


@pytest.mark.parametrize("seg_num,seg_len,k,period", [(1500, 8000, 50, 1024), (800, 4096, 64, 2048)])
def test_periodic_f32(seg_num, seg_len, k, period):
    from tests.test_f32_gpu import run_f32

    bits = _periodic(seg_num * seg_len, period, fmt="f32").reshape(seg_num, seg_len)
    exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS, fmt="f32")
    announce(f"periodic f32 {seg_num}x{seg_len} k={k} period={period}")
    assert_same(run_f32(bits, k, elem_offset=2), exp, f"periodic f32 {seg_num}x{seg_len}")
