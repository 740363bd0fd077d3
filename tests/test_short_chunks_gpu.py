"""GPU parity of short chunks against the oracle.

A chunk whose positions all sit in each thread's first vector, with at most 4 * EV * kc of them
(EV = elements per 16-byte load), takes its threshold from an LDS histogram of its elements
instead of its thread bests (the SHORT kernel instantiations, chosen at launch for segmented
input and for short fixed-length rows).  These cases cover both layouts and every element
format, with data that drives each branch after the threshold: the positive and non-positive
filters, the all-elements path (the kc-th key is a NaN), ties at the threshold, and the overflow
refinement (more tied elements than the candidate list holds)."""

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


def _f16_rows(kind, rng, shape):
    n = int(np.prod(shape))
    if kind == "normal":
        x = rng.standard_normal(n).astype(np.float16).view(np.uint16)
    elif kind == "negative":
        x = (-np.abs(rng.standard_normal(n)) - 0.1).astype(np.float16).view(np.uint16)
    elif kind == "ties":
        x = (rng.integers(-2, 3, size=n) * 0.5).astype(np.float16).view(np.uint16)
    elif kind == "all_equal":
        x = np.full(n, 0xBC00, dtype=np.uint16)                      # -1.0 everywhere
    elif kind == "nan_heavy":
        x = rng.standard_normal(n).astype(np.float16).view(np.uint16)
        x[rng.random(n) < 0.9] = 0x7E00
    else:
        raise KeyError(kind)
    return x.reshape(shape)


KINDS = ["normal", "negative", "ties", "all_equal", "nan_heavy"]


@pytest.mark.parametrize("seg_num,seg_len,k", [(64, 300, 64), (16, 1000, 300), (7, 2047, 512),
                                               (33, 65, 64), (5, 8, 8), (12, 4096, 200)])
@pytest.mark.parametrize("kind", KINDS)
def test_short_fixed_rows_f16(seg_num, seg_len, k, kind):
    rng = np.random.default_rng(seg_num * 1000 + seg_len + k)
    bits = _f16_rows(kind, rng, (seg_num, seg_len))
    for elem_offset in (0, 5):
        announce(f"short fixed f16 {kind} {seg_num}x{seg_len} k={k} offset={elem_offset}")
        got = run_fixed(bits, k, elem_offset=elem_offset, poison=0x3C)
        exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS)
        assert_same(got, exp, f"short fixed f16 {kind}")


@pytest.mark.parametrize("kind", KINDS)
def test_short_fixed_rows_bf16(kind):
    rng = np.random.default_rng(7)
    f = _f16_rows(kind, rng, (40, 700)).view(np.float16).astype(np.float32)
    bf = (f.view(np.uint32) >> 16).astype(np.uint16)
    if kind == "nan_heavy":
        bf[np.isnan(f)] = 0x7FC1
    announce(f"short fixed bf16 {kind}")
    got = run_fixed(bf, 96, fmt="bf16")
    exp = O.batch_topk_half(bf, 96, seg_len=700, threads=THREADS, fmt="bf16")
    assert_same(got, exp, f"short fixed bf16 {kind}")


@pytest.mark.parametrize("kind", KINDS)
def test_short_fixed_rows_f32(kind):
    import torch

    rng = np.random.default_rng(8)
    f = _f16_rows(kind, rng, (24, 900)).view(np.float16).astype(np.float32)
    bits = f.view(np.uint32).copy()
    bits[np.isnan(f)] = 0x7FC00001
    x = torch.from_numpy(bits.view(np.float32)).to("cuda:0")
    announce(f"short fixed f32 {kind}")
    v, i = bt.topk(x, 128)
    torch.cuda.synchronize()
    exp = O.batch_topk_half(bits, 128, seg_len=900, threads=THREADS, fmt="f32")
    assert np.array_equal(i.cpu().numpy(), exp[1]), kind
    assert np.array_equal(v.cpu().numpy().view(np.uint32), exp[0]), kind


def test_short_negative_segments():
    # every segment short and negative: the non-positive-threshold filter and the
    # all-elements path over chunks that are mostly past their segment's end
    rng = np.random.default_rng(9)
    lengths = rng.integers(1, 600, size=700).astype(np.int64)
    lengths[::7] = rng.integers(60000, 65536, size=lengths[::7].size)   # some long ones
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    bits = (-np.abs(rng.standard_normal(int(offsets[-1]))) - 0.01).astype(np.float16).view(np.uint16)
    for k in (1, 64, 300):
        announce(f"short negative segments k={k}")
        got = run_segmented(bits, offsets, k, 65536, elem_offset=3, poison=0x5A)
        exp = O.batch_topk_half(bits, k, offsets=offsets.astype(np.int64), threads=THREADS)
        assert_same(got, exp, f"short negative segments k={k}")
