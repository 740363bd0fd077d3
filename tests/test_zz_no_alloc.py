"""GPU test of radix_topk_batch_topk_half_noalloc against radix_topk_batch_topk_half.

The allocation-free entry point runs the same kernels with the library's static per-GPU
workspace.  Two calls in a row on the same GPU (the second on a smaller input, so the array
holds the first call's words when the second starts) must each give the plain entry point's
results bit for bit, on every plan kind: one chunk per segment, the two-chunk merge, the
cooperative grid and the long-segment path."""

import numpy as np
import pytest

import batch_topk_amd as bt
from tests.gpu_util import announce, assert_same, run_fixed

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    bt.load_library()


def run_noalloc(bits, k):
    import torch

    seg_num, seg_len = bits.shape
    x = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to("cuda:0")
    vals = torch.full((seg_num, k), 0x1234, dtype=torch.int16, device="cuda:0")
    idx = torch.full((seg_num, k), -7, dtype=torch.int32, device="cuda:0")
    rc = bt.batch_topk_half_noalloc(x.data_ptr(), seg_num, seg_len, k, vals.data_ptr(), idx.data_ptr(),
                                    torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return vals.cpu().numpy().view(np.uint16), idx.cpu().numpy()


# (larger, smaller) pairs of calls in a row
PAIRS = [
    ((128, 128256, 50), (16, 4096, 50)),        # one chunk per segment
    ((64, 200000, 50), (8, 150000, 16)),        # the two-chunk merge
    ((1, 1 << 24, 1024), (1, 1_000_000, 300)),  # the cooperative grid
    ((1, 40_000_000, 64), (2, 20_000_000, 8)),  # the long-segment path
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_plain_entry_point(first, second):
    rng = np.random.default_rng(first[1])
    for seg_num, seg_len, k in (first, second):
        bits = rng.standard_normal((seg_num, seg_len), dtype=np.float32).astype(np.float16).view(np.uint16)
        announce(f"noalloc {seg_num}x{seg_len} k={k}")
        got = run_noalloc(bits, k)
        exp = run_fixed(bits, k, poison=0xA5)
        assert_same(got, exp, f"noalloc {seg_num}x{seg_len} k={k}")
