"""GPU parity of segments split over two workgroups (two chunks), against the oracle.

The two workgroups of such a segment meet once: the first to take the segment's ticket
publishes its chunk's list with words tagged for the call, the second polls for it, merges and
clears what it consumed.  These tests reuse one workspace across calls with new data (stale
lists must never be taken for fresh ones) and replay a captured HIP graph, whose every replay
carries the same call epoch."""

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


def _rows(kind, rng, seg_num, seg_len):
    if kind == "normal":
        return rng.standard_normal((seg_num, seg_len)).astype(np.float16).view(np.uint16)
    if kind == "ties":
        return (rng.integers(-3, 4, size=(seg_num, seg_len)) * 0.5).astype(np.float16).view(np.uint16)
    if kind == "sorted":
        x = np.sort(rng.standard_normal((seg_num, seg_len)).astype(np.float16), axis=1)
        return x.view(np.uint16)
    if kind == "nan_rows":
        x = rng.standard_normal((seg_num, seg_len)).astype(np.float16).view(np.uint16)
        x[::2] = 0x7E00 | (np.arange(seg_len, dtype=np.uint16) & 0xff)  # whole rows of NaN
        return x
    if kind == "top_in_one_chunk":
        # every large value in the second half: the first chunk's list holds none of the result
        x = rng.standard_normal((seg_num, seg_len)).astype(np.float16)
        x[:, seg_len // 2:] += np.float16(8.0)
        return x.view(np.uint16)
    raise KeyError(kind)


# (seg_num, seg_len, k): rows of 131,066..262,137 elements take two 131,072-element chunks
# (k up to 512 keeps both lists within one workgroup's merge); the tail chunk ranges from a
# few elements to almost a full chunk.
PAIR_SHAPES = [
    (64, 200000, 50),
    (128, 140000, 50),
    (16, 250000, 1),
    (12, 180000, 128),
    (8, 200000, 256),
    (3, 250000, 512),
    (600, 65536, 64),  # 512-thread chunks of 65,536: misaligned rows leave a tail of <= 7
]


@pytest.mark.parametrize("seg_num,seg_len,k", PAIR_SHAPES)
def test_two_chunk_segments_repeated_on_one_workspace(seg_num, seg_len, k):
    torch = pytest.importorskip("torch")
    ws = torch.empty(bt.batch_topk_half_workspace_size(seg_num, seg_len, k), dtype=torch.uint8,
                     device="cuda:0")
    ws.fill_(0xA5)
    rng = np.random.default_rng(seg_len + k)
    for rep, kind in enumerate(["normal", "ties", "top_in_one_chunk", "sorted", "nan_rows", "normal"]):
        bits = _rows(kind, rng, seg_num, seg_len)
        elem_offset = rep % 3 * 3
        announce(f"two-chunk {seg_num}x{seg_len} k={k} rep={rep} {kind} offset={elem_offset}")
        got = run_fixed(bits, k, workspace=ws, elem_offset=elem_offset)
        exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS)
        assert_same(got, exp, f"two-chunk {kind} rep {rep}")


def test_two_chunk_bf16_and_segmented_mix():
    # segmented input whose plan has three chunks: segments of one, two (pair merge) and
    # three chunks (last-arriver merge) in one call, with fresh data twice
    rng = np.random.default_rng(77)
    lengths = np.array([300000, 131000, 200000, 5, 0, 140000, 262000, 131072, 90000], dtype=np.int64)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    for rep in range(2):
        bits = rng.standard_normal(int(offsets[-1])).astype(np.float16).view(np.uint16)
        for k in (64, 200):
            announce(f"segmented mix rep={rep} k={k}")
            got = run_segmented(bits, offsets, k, 300000, poison=0x5A)
            exp = O.batch_topk_half(bits, k, offsets=offsets.astype(np.int64), threads=THREADS)
            assert_same(got, exp, f"segmented mix k={k}")
    bits = rng.standard_normal((32, 150000)).astype(np.float32)
    bf = (bits.view(np.uint32) >> 16).astype(np.uint16)  # bf16 patterns by truncation
    announce("two-chunk bf16 32x150000 k=50")
    got = run_fixed(bf, 50, fmt="bf16")
    exp = O.batch_topk_half(bf, 50, seg_len=150000, threads=THREADS, fmt="bf16")
    assert_same(got, exp, "two-chunk bf16")


def test_two_chunk_graph_replays():
    # A captured call replays with its epoch frozen; new input between replays, and eager calls
    # on the same workspace in between, must still give fresh results every time.
    torch = pytest.importorskip("torch")
    seg_num, seg_len, k = 64, 200000, 50
    rng = np.random.default_rng(2024)
    x = torch.empty((seg_num, seg_len), dtype=torch.float16, device="cuda:0")
    ws = torch.empty(bt.batch_topk_half_workspace_size(seg_num, seg_len, k), dtype=torch.uint8,
                     device="cuda:0")
    ws.fill_(0)

    def fresh():
        bits = _rows("normal" if rng.integers(0, 2) else "ties", rng, seg_num, seg_len)
        x.copy_(torch.from_numpy(bits.view(np.float16)).to("cuda:0"))
        torch.cuda.synchronize()
        return bits

    bits = fresh()
    announce("graph capture 64x200000 k=50")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        vals, idx = bt.topk(x, k, workspace=ws)
    for rep in range(4):
        bits = fresh()
        announce(f"graph replay {rep}")
        g.replay()
        torch.cuda.synchronize()
        exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS)
        got = (vals.view(torch.int16).cpu().numpy().view(np.uint16), idx.cpu().numpy())
        assert_same(got, exp, f"graph replay {rep}")
        # an eager call on the same workspace between replays
        v2, i2 = bt.topk(x, k, workspace=ws)
        torch.cuda.synchronize()
        assert_same((v2.view(torch.int16).cpu().numpy().view(np.uint16), i2.cpu().numpy()), exp,
                    f"eager call after replay {rep}")
