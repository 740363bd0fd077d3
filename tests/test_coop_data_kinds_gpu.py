"""GPU parity of the cooperative (whole-segment) path across data kinds.

Long segments with large k run as one grid of co-resident workgroups, one per 65,536-element
chunk, that agree on a whole-segment threshold and rank one whole-segment candidate list.
How many elements pass the threshold, and how they spread over the chunks, depends on the
data: these tests compare the path with the oracle on normal rows, heavy ties (lists past the
LDS capacity, so the exact refinement runs), ascending and descending rows (every top value in
the last or the first chunk), NaN/+-inf mixes, a last chunk of 5 elements, bfloat16 rows and a
segmented batch whose rows span from one chunk to nineteen, each on a workspace poisoned before
the call."""

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


def _data(kind, rng, n, fmt="f16"):
    if kind == "normal":
        x = rng.standard_normal(n, dtype=np.float32)
    elif kind == "ties":  # 13 distinct values
        x = (rng.integers(-6, 7, size=n) * 0.25).astype(np.float32)
    elif kind == "sorted":  # every top value in the last chunk
        x = np.sort(rng.standard_normal(n, dtype=np.float32))
    elif kind == "descending":  # every top value in the first chunk
        x = -np.sort(rng.standard_normal(n, dtype=np.float32))
    elif kind == "nan_inf":  # NaNs, -inf and a few +inf among normals
        x = rng.standard_normal(n, dtype=np.float32)
        r = rng.random(n)
        x[r < 0.3] = np.nan
        x[(r >= 0.3) & (r < 0.5)] = -np.inf
        x[r > 0.99995] = np.inf
    else:
        raise KeyError(kind)
    if fmt == "bf16":
        import torch

        return torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    return x.astype(np.float16).view(np.uint16)


# (seg_num, seg_len, k, kind): every shape plans as a cooperative grid of 8-vector chunks.
CASES = [
    (1, 16_777_216, 1024, "normal"),       # 256 chunks
    (1, 1_000_000, 1024, "normal"),        # 16 chunks
    (1, 1_000_000, 1024, "ties"),          # lists past the LDS capacity: exact refinement
    (1, 1_000_000, 1024, "sorted"),
    (1, 1_000_000, 1024, "descending"),
    (1, 1_000_000, 1024, "nan_inf"),
    (1, 4_000_000, 512, "normal"),
    (2, 3_000_000, 64, "normal"),
    (1, 3_000_000, 8, "normal"),
    (4, 600_000, 300, "normal"),
    (4, 600_000, 300, "ties"),
    (1, 65536 * 20 + 5, 256, "normal"),    # a last chunk of 5 elements
    (1, 65536 * 20 + 5, 256, "nan_inf"),
]


@pytest.mark.parametrize("seg_num,seg_len,k,kind", CASES)
def test_coop_parity(seg_num, seg_len, k, kind):
    rng = np.random.default_rng(seg_len + k)
    bits = _data(kind, rng, seg_num * seg_len).reshape(seg_num, seg_len)
    exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS)
    announce(f"cooperative {seg_num}x{seg_len} k={k} {kind}")
    assert_same(run_fixed(bits, k, poison=0xA5), exp, f"{kind} {seg_num}x{seg_len} k={k}")


@pytest.mark.parametrize("seg_num,seg_len,k,kind", [(1, 2_000_000, 500, "normal"), (1, 2_000_000, 500, "nan_inf")])
def test_coop_parity_bf16(seg_num, seg_len, k, kind):
    rng = np.random.default_rng(7)
    bits = _data(kind, rng, seg_num * seg_len, fmt="bf16").reshape(seg_num, seg_len)
    exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS, fmt="bf16")
    announce(f"cooperative bf16 {seg_num}x{seg_len} k={k} {kind}")
    assert_same(run_fixed(bits, k, poison=0x5A, fmt="bf16"), exp, f"bf16 {kind}")


def test_coop_segmented():
    # rows of 1 to 19 chunks, one with a 3-element last chunk, and an empty row
    rng = np.random.default_rng(11)
    lengths = [1_200_000, 65536 * 5 + 3, 900_000, 40_000, 0, 777_777]
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    bits = _data("normal", rng, int(offsets[-1]))
    k, max_len = 500, max(lengths)
    exp = O.batch_topk_half(bits, k, offsets=offsets, threads=THREADS)
    announce(f"cooperative segmented {lengths} k={k}")
    assert_same(run_segmented(bits, offsets, k, max_len, poison=0xA5), exp, "segmented")
