"""GPU parity of the long-segment path against the oracle.

Segments whose whole-segment threshold needs more single-chunk workgroups than the CUs hold at
once (a segment longer than 256 chunks of 131,072 fp16 elements, or many long segments with
large k) are split over `group` workgroups per segment, each taking several chunks.  With one
workgroup per segment (many segments) nothing crosses workgroups.  The shapes here all
returned workspace 0 before this path existed (the reference's own envelope is
seg_len <= 10000, k <= 128: src/batch_topk.cu:13-16)."""

import numpy as np
import pytest

import batch_topk_amd as bt
from oracle import oracle as O
from tests.gpu_util import announce, assert_properties, assert_same, run_fixed, run_segmented

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


def _bits(kind, rng, n):
    if kind == "normal":
        return rng.standard_normal(n, dtype=np.float32).astype(np.float16).view(np.uint16)
    if kind == "ties":
        return (rng.integers(-3, 4, size=n) * 0.5).astype(np.float16).view(np.uint16)
    if kind == "sorted":
        return np.sort(rng.standard_normal(n, dtype=np.float32).astype(np.float16)).view(np.uint16)
    raise KeyError(kind)


@pytest.mark.parametrize("seg_num,seg_len,k,kind,elem_offset", [
    (1, 50_000_000, 1, "normal", 0),
    (1, 50_000_000, 1024, "normal", 3),
    (4, 20_000_000, 64, "normal", 1),
    (1, 40_000_000, 1024, "ties", 0),       # every workgroup's list overflows: the refinement
    (2, 20_000_000, 300, "sorted", 5),      # the top of each row in its last chunks
])
def test_long_fixed_segments(seg_num, seg_len, k, kind, elem_offset):
    rng = np.random.default_rng(seg_len + k)
    bits = _bits(kind, rng, seg_num * seg_len).reshape(seg_num, seg_len)
    announce(f"long segments {seg_num}x{seg_len} k={k} {kind} offset={elem_offset}")
    got = run_fixed(bits, k, poison=0xA5, elem_offset=elem_offset)
    exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS)
    assert_same(got, exp, f"long {seg_num}x{seg_len} k={k} {kind}")
    assert_properties(bits, got[0], got[1], k, [seg_len] * seg_num)


@pytest.mark.parametrize("kind", ["normal", "ties"])
def test_one_workgroup_per_long_segment(kind):
    # more segments than CUs, each longer than one chunk, k large: one workgroup per segment
    # takes both of its chunks and selects alone
    rng = np.random.default_rng(17)
    seg_num, seg_len, k = 300, 200_000, 1024
    bits = _bits(kind, rng, seg_num * seg_len).reshape(seg_num, seg_len)
    announce(f"one workgroup per segment {seg_num}x{seg_len} k={k} {kind}")
    got = run_fixed(bits, k, elem_offset=2)
    assert_same(got, O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS), f"solo {kind}")


def test_long_segmented_218_segments():
    # 218 variable segments of up to 131,072 (two chunks each when misaligned), k = 1024
    rng = np.random.default_rng(218)
    lengths = rng.integers(0, 131073, size=218).astype(np.int64)
    lengths[:6] = [131072, 131072, 0, 1, 1023, 131071]
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    bits = _bits("normal", rng, int(offsets[-1]))
    bits[offsets[0]:offsets[0] + 40_000] = 0x3C00  # a long run of equal values in segment 0
    assert bt.batch_topk_half_segmented_workspace_size(218, 131072, 1024) > 0
    for elem_offset in (0, 5):
        announce(f"long segmented 218 x <=131072 k=1024 offset={elem_offset}")
        got = run_segmented(bits, offsets, 1024, 131072, poison=0x5A, elem_offset=elem_offset)
        exp = O.batch_topk_half(bits, 1024, offsets=offsets.astype(np.int64), threads=THREADS)
        assert_same(got, exp, f"long segmented offset={elem_offset}")


def test_long_f32_rows():
    import torch

    rng = np.random.default_rng(32)
    for seg_num, seg_len, k, off in ((1, (1 << 24) + 1, 1024, 1), (2, 1 << 24, 512, 0)):
        x = rng.standard_normal(seg_num * seg_len, dtype=np.float32)
        bits = x.view(np.uint32).reshape(seg_num, seg_len)
        ws_bytes = bt.batch_topk_f32_workspace_size(seg_num, seg_len, k)
        assert ws_bytes > 0
        host = np.zeros(seg_num * seg_len + off + 4, dtype=np.uint32)
        host[off:off + seg_num * seg_len] = bits.reshape(-1)
        buf = torch.from_numpy(host.view(np.int32)).to("cuda:0")
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
        vals = torch.empty((seg_num, k), dtype=torch.int32, device="cuda:0")
        idx = torch.empty((seg_num, k), dtype=torch.int32, device="cuda:0")
        announce(f"long fp32 {seg_num}x{seg_len} k={k} offset={off}")
        rc = bt.batch_topk_f32(buf.data_ptr() + 4 * off, seg_num, seg_len, k, vals.data_ptr(), idx.data_ptr(),
                               ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS, fmt="f32")
        assert_same((vals.cpu().numpy().view(np.uint32), idx.cpu().numpy()), exp, f"long fp32 {seg_num}x{seg_len}")


def test_long_graph_replays_and_status():
    torch = pytest.importorskip("torch")
    seg_num, seg_len, k = 1, 36_000_000, 300
    rng = np.random.default_rng(36)
    x = torch.empty((seg_num, seg_len), dtype=torch.float16, device="cuda:0")
    ws_bytes = bt.batch_topk_half_workspace_size(seg_num, seg_len, k)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
    ws.fill_(0xA5)

    def fresh(kind):
        bits = _bits(kind, rng, seg_num * seg_len).reshape(seg_num, seg_len)
        x.copy_(torch.from_numpy(bits.view(np.float16)).to("cuda:0"))
        torch.cuda.synchronize()
        return bits

    fresh("normal")
    announce("long-segment graph capture 1x36000000 k=300")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        vals, idx = bt.topk(x, k, workspace=ws)
    for rep, kind in enumerate(["normal", "ties", "normal"]):
        bits = fresh(kind)
        announce(f"long-segment graph replay {rep} ({kind})")
        g.replay()
        torch.cuda.synchronize()
        exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS)
        assert_same((vals.view(torch.int16).cpu().numpy().view(np.uint16), idx.cpu().numpy()), exp,
                    f"long replay {rep}")
        assert bt.workspace_status(ws.data_ptr(), ws_bytes, seg_num) == [bt.STATUS_OK]
        v2, i2 = bt.topk(x, k, workspace=ws)
        torch.cuda.synchronize()
        assert_same((v2.view(torch.int16).cpu().numpy().view(np.uint16), i2.cpu().numpy()), exp,
                    f"long eager after replay {rep}")


@pytest.mark.parametrize("force", [1, 2, 4])
def test_long_forced_wait_timeouts(force):
    torch = pytest.importorskip("torch")
    seg_num, seg_len, k = 1, 36_000_000, 300
    rng = np.random.default_rng(force)
    bits = _bits("normal", rng, seg_num * seg_len).reshape(seg_num, seg_len)
    x = torch.from_numpy(bits.view(np.float16)).to("cuda:0")
    ws_bytes = bt.batch_topk_half_workspace_size(seg_num, seg_len, k)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
    ws.fill_(0)
    announce(f"long forced timeout {force}")
    bt.debug_wait_hook(64, force)
    try:
        v, i = bt.topk(x, k, workspace=ws)
        torch.cuda.synchronize()
    finally:
        bt.debug_wait_hook(0, 0)
    assert bt.workspace_status(ws.data_ptr(), ws_bytes, seg_num) == [bt.STATUS_WAIT_TIMEOUT]
    assert np.all(i.cpu().numpy() == bt.PAD_INDEX)
    announce(f"long forced timeout {force}: ordinary call after it")
    v, i = bt.topk(x, k, workspace=ws)
    torch.cuda.synchronize()
    exp = O.batch_topk_half(bits, k, seg_len=seg_len, threads=THREADS)
    assert_same((v.view(torch.int16).cpu().numpy().view(np.uint16), i.cpu().numpy()), exp, "after timeout")
    assert bt.workspace_status(ws.data_ptr(), ws_bytes, seg_num) == [bt.STATUS_OK]
