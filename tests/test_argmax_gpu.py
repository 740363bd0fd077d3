"""GPU parity of k = 1 (the row's best element: value and smallest index among ties) against the
oracle.  Single-chunk 16-bit rows take a path of their own (two workgroup minima, no candidate
list): these rows cover what it must get right -- ties, NaNs of either sign next to the best value
(a thread whose int16 maximum is a positive NaN reports a worse thread best), +inf, rows of no
positive value (which take the general path), every alignment, fp16 and bf16."""

import numpy as np
import pytest

import batch_topk_amd as bt
from oracle import oracle as O
from tests.gpu_util import announce, assert_same, run_fixed

pytestmark = pytest.mark.gpu

THREADS = 8


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    bt.load_library()


def _rows(kind, rng, seg_num, seg_len, fmt):
    if fmt == "f16":
        def bits_of(x):
            return x.astype(np.float16).view(np.uint16)
        nan_pos, nan_neg, pinf = 0x7E00, 0xFE01, 0x7C00
    else:
        def bits_of(x):
            return (x.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        nan_pos, nan_neg, pinf = 0x7FC0, 0xFF81, 0x7F80
    if kind == "normal":
        return bits_of(rng.standard_normal((seg_num, seg_len)))
    if kind == "ties":
        return bits_of(rng.integers(-8, 9, size=(seg_num, seg_len)) * 0.25)
    if kind == "nan_neighbours":
        x = bits_of(rng.standard_normal((seg_num, seg_len)))
        flat = x.reshape(-1)
        flat[rng.integers(0, flat.size, size=flat.size // 16)] = nan_pos   # in most vectors
        flat[rng.integers(0, flat.size, size=flat.size // 64)] = nan_neg
        return x
    if kind == "inf_and_nan":
        x = bits_of(rng.standard_normal((seg_num, seg_len)))
        for r in range(seg_num):
            x[r, rng.integers(0, seg_len, size=3)] = pinf
            x[r, rng.integers(0, seg_len, size=5)] = nan_pos
        return x
    if kind == "negative":
        return bits_of(-np.abs(rng.standard_normal((seg_num, seg_len))) - 0.5)
    if kind == "zeros_and_negative":
        x = bits_of(-np.abs(rng.standard_normal((seg_num, seg_len))))
        x[:, ::7] = 0x8000
        x[:, 3::11] = 0x0000
        return x
    if kind == "all_nan":
        return np.full((seg_num, seg_len), nan_pos, dtype=np.uint16)
    raise KeyError(kind)


@pytest.mark.parametrize("fmt", ["f16", "bf16"])
@pytest.mark.parametrize("kind", ["normal", "ties", "nan_neighbours", "inf_and_nan", "negative",
                                  "zeros_and_negative", "all_nan"])
@pytest.mark.parametrize("seg_num,seg_len", [(256, 32000), (128, 128256), (16, 4096), (40, 65536), (3, 777)])
def test_k1_rows(seg_num, seg_len, kind, fmt):
    rng = np.random.default_rng(seg_num * 31 + seg_len + len(kind))
    bits = _rows(kind, rng, seg_num, seg_len, fmt)
    for elem_offset in (0, 5):
        announce(f"k=1 {fmt} {kind} {seg_num}x{seg_len} offset={elem_offset}")
        got = run_fixed(bits, 1, elem_offset=elem_offset, fmt=fmt, poison=0xA5)
        exp = O.batch_topk_half(bits, 1, seg_len=seg_len, threads=THREADS, fmt=fmt)
        assert_same(got, exp, f"k=1 {fmt} {kind} {seg_num}x{seg_len} offset={elem_offset}")
