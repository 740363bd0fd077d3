"""GPU tests of the cross-workgroup protocols under HIP-graph replay and under bounded waits
that give up.

Long segments with large k run as one grid whose workgroups meet through the workspace.  A
captured call replays with its host-side call epoch frozen, so every word the workgroups
exchange carries a token that also mixes in a per-segment generation word the call advances:
these tests replay captured calls with new input between replays and eager calls on the same
workspace in between, and check every result against the oracle.

Every cross-workgroup wait is bounded.  The test hook radix_topk_debug_wait_hook makes a
chosen wait look for a value no workgroup writes, with a small spin limit: the wait gives up,
the segment's row gets the pad and its status word RADIX_TOPK_STATUS_WAIT_TIMEOUT, and every
kernel still runs to its end.  The next ordinary call on the same workspace must be correct
and report RADIX_TOPK_STATUS_OK."""

import numpy as np
import pytest

import batch_topk_amd as bt
from oracle import oracle as O
from tests.gpu_util import announce, assert_same

pytestmark = pytest.mark.gpu

THREADS = 8


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    bt.load_library()
    yield
    bt.debug_wait_hook(0, 0)


def _rows(kind, rng, n):
    if kind == "normal":
        return rng.standard_normal(n).astype(np.float16).view(np.uint16)
    if kind == "ties":
        return (rng.integers(-6, 7, size=n) * 0.25).astype(np.float16).view(np.uint16)
    if kind == "sorted":
        return np.sort(rng.standard_normal(n).astype(np.float16)).view(np.uint16)
    raise KeyError(kind)


def _bits_of(t):
    import torch

    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def _fixed_graph_replays(seg_num, seg_len, k, kinds, seed):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(seed)
    x = torch.empty((seg_num, seg_len), dtype=torch.float16, device="cuda:0")
    ws_bytes = bt.batch_topk_half_workspace_size(seg_num, seg_len, k)
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
    ws.fill_(0xA5)

    def fresh(kind):
        bits = _rows(kind, rng, seg_num * seg_len).reshape(seg_num, seg_len)
        x.copy_(torch.from_numpy(bits.view(np.float16)).to("cuda:0"))
        torch.cuda.synchronize()
        return bits

    fresh("normal")
    announce(f"cooperative graph capture {seg_num}x{seg_len} k={k}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        vals, idx = bt.topk(x, k, workspace=ws)
    for rep, kind in enumerate(kinds):
        bits = fresh(kind)
        announce(f"cooperative graph replay {rep} ({kind}) {seg_num}x{seg_len} k={k}")
        g.replay()
        torch.cuda.synchronize()
        exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS)
        assert_same((_bits_of(vals), idx.cpu().numpy()), exp, f"graph replay {rep} ({kind})")
        assert bt.workspace_status(ws.data_ptr(), ws_bytes, seg_num) == [bt.STATUS_OK] * seg_num
        # an eager call on the same workspace between replays
        v2, i2 = bt.topk(x, k, workspace=ws)
        torch.cuda.synchronize()
        assert_same((_bits_of(v2), i2.cpu().numpy()), exp, f"eager call after replay {rep}")
        assert bt.workspace_status(ws.data_ptr(), ws_bytes, seg_num) == [bt.STATUS_OK] * seg_num


@pytest.mark.parametrize("seg_num,seg_len,k", [(1, 1_000_000, 1024), (3, 300_001, 512)])
def test_cooperative_graph_replays(seg_num, seg_len, k):
    _fixed_graph_replays(seg_num, seg_len, k, ["normal", "ties", "sorted", "normal", "ties"], seg_len)


def test_cooperative_graph_replays_huge_segment():
    # the single 2^24-element segment with k = 1024 (one workgroup per 131,072 elements)
    _fixed_graph_replays(1, 1 << 24, 1024, ["normal", "ties", "normal", "normal"], 24)


def test_cooperative_segmented_graph_replays():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(37)
    lengths = np.array([400_000, 5, 0, 300_000, 150_000, 131_072, 131_073], dtype=np.int64)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    seg_num, max_len, k = lengths.size, 400_000, 300
    n = int(offsets[-1])
    x = torch.empty(n, dtype=torch.float16, device="cuda:0")
    d_off = torch.from_numpy(offsets).to("cuda:0")
    ws_bytes = bt.batch_topk_half_segmented_workspace_size(seg_num, max_len, k)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
    ws.fill_(0x5A)

    def fresh(kind):
        bits = _rows(kind, rng, n)
        bits[offsets[3]:offsets[3] + 50_000] = 0x3C00
        x.copy_(torch.from_numpy(bits.view(np.float16)).to("cuda:0"))
        torch.cuda.synchronize()
        return bits

    fresh("normal")
    announce("cooperative segmented graph capture k=300")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        vals, idx = bt.segmented_topk(x, d_off, k, max_len, workspace=ws)
    for rep, kind in enumerate(["normal", "ties", "sorted", "normal"]):
        bits = fresh(kind)
        announce(f"cooperative segmented graph replay {rep} ({kind})")
        g.replay()
        torch.cuda.synchronize()
        exp = O.batch_topk_half(bits, k, offsets=offsets.astype(np.int64), threads=THREADS)
        assert_same((_bits_of(vals), idx.cpu().numpy()), exp, f"segmented replay {rep}")
        v2, i2 = bt.segmented_topk(x, d_off, k, max_len, workspace=ws)
        torch.cuda.synchronize()
        assert_same((_bits_of(v2), i2.cpu().numpy()), exp, f"segmented eager after replay {rep}")
        assert bt.workspace_status(ws.data_ptr(), ws_bytes, seg_num) == [bt.STATUS_OK] * seg_num


# (force bit, shape): the long-segment grid's first wait, first meeting and list collection, and
# the two-chunk merger's poll.
FORCED = [
    (1, (1, 1_000_000, 1024)),
    (2, (1, 1_000_000, 1024)),
    (4, (2, 600_000, 300)),
    (8, (16, 200_000, 50)),
]


@pytest.mark.parametrize("force,shape", FORCED)
def test_forced_wait_timeouts_report_status(force, shape):
    torch = pytest.importorskip("torch")
    seg_num, seg_len, k = shape
    rng = np.random.default_rng(force)
    bits = _rows("normal", rng, seg_num * seg_len).reshape(seg_num, seg_len)
    x = torch.from_numpy(bits.view(np.float16)).to("cuda:0")
    ws_bytes = bt.batch_topk_half_workspace_size(seg_num, seg_len, k)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
    ws.fill_(0)
    exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS)
    # an ordinary call first: complete rows, status OK
    announce(f"forced timeout {force}: ordinary call {shape}")
    v, i = bt.topk(x, k, workspace=ws)
    torch.cuda.synchronize()
    assert_same((_bits_of(v), i.cpu().numpy()), exp, "before the forced timeout")
    assert bt.workspace_status(ws.data_ptr(), ws_bytes, seg_num) == [bt.STATUS_OK] * seg_num
    # the forced timeout: every wait of that kind gives up after 64 polls
    announce(f"forced timeout {force}: forced call {shape}")
    bt.debug_wait_hook(64, force)
    try:
        v, i = bt.topk(x, k, workspace=ws)
        torch.cuda.synchronize()
    finally:
        bt.debug_wait_hook(0, 0)
    assert bt.workspace_status(ws.data_ptr(), ws_bytes, seg_num) == [bt.STATUS_WAIT_TIMEOUT] * seg_num
    assert np.all(i.cpu().numpy() == bt.PAD_INDEX)
    assert np.all(_bits_of(v) == bt.PAD_VALUE_BITS)
    # the next ordinary calls on the same workspace are complete and correct
    for rep in range(2):
        announce(f"forced timeout {force}: ordinary call {rep} after it")
        v, i = bt.topk(x, k, workspace=ws)
        torch.cuda.synchronize()
        assert_same((_bits_of(v), i.cpu().numpy()), exp, f"after the forced timeout {rep}")
        assert bt.workspace_status(ws.data_ptr(), ws_bytes, seg_num) == [bt.STATUS_OK] * seg_num


def test_status_of_every_plan_kind():
    # one chunk, two chunks (pair merge), three chunks (last arriver), cooperative
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    for seg_num, seg_len, k in ((64, 20000, 50), (16, 200000, 50), (4, 300000, 16), (2, 500000, 700)):
        bits = _rows("normal", rng, seg_num * seg_len).reshape(seg_num, seg_len)
        x = torch.from_numpy(bits.view(np.float16)).to("cuda:0")
        ws_bytes = bt.batch_topk_half_workspace_size(seg_num, seg_len, k)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
        ws.fill_(0xFF)  # every status word starts as garbage
        announce(f"status {seg_num}x{seg_len} k={k}")
        v, i = bt.topk(x, k, workspace=ws)
        torch.cuda.synchronize()
        assert_same((_bits_of(v), i.cpu().numpy()), O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS),
                    f"status {seg_num}x{seg_len}")
        assert bt.workspace_status(ws.data_ptr(), ws_bytes, seg_num) == [bt.STATUS_OK] * seg_num
