"""GPU parity of radix_topk_batch_topk_ex: every layout, format and output flag against the
oracle (and the plain entry points against the same oracle rows).

flags = 0 must give the oracle's rows bit for bit; UNSORTED must give, in each row's first
min(k, length) slots, the oracle row's set of (index, value bits) entries, and the pad after
them; INDICES_ONLY must give the oracle's indices and leave the value array untouched."""

import numpy as np
import pytest

import batch_topk_amd as bt
from oracle import oracle as O
from tests.gpu_util import announce, assert_same, device_u16, run_fixed, run_segmented

pytestmark = pytest.mark.gpu

THREADS = 8
SENTINEL = 0x1234


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    bt.load_library()


def run_ex(bits, k, flags, fmt=bt.FORMAT_F16, offsets=None, max_len=None):
    """radix_topk_batch_topk_ex on fixed rows [seg_num, seg_len] or a flat array with offsets."""
    import torch

    if offsets is None:
        seg_num, seg_len = bits.shape
    else:
        seg_num, seg_len = offsets.size - 1, max_len
    buf = device_u16(bits)
    d_off = torch.from_numpy(offsets.astype(np.int32)).to("cuda:0") if offsets is not None else None
    ws_bytes = bt.batch_topk_ex_workspace_size(fmt, offsets is not None, seg_num, seg_len, k)
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
    ws.fill_(0xC3)
    vals = torch.full((seg_num, k), SENTINEL, dtype=torch.int16, device="cuda:0")
    idx = torch.full((seg_num, k), -7, dtype=torch.int32, device="cuda:0")
    indices_only = bool(flags & bt.INDICES_ONLY)
    rc = bt.batch_topk_ex(buf.data_ptr(), fmt, d_off.data_ptr() if d_off is not None else 0, seg_num,
                          seg_len, k, flags, 0 if indices_only else vals.data_ptr(), idx.data_ptr(),
                          ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return vals.cpu().numpy().view(np.uint16), idx.cpu().numpy()


def check_variants(bits, k, what, fmt=bt.FORMAT_F16, offsets=None, max_len=None):
    fmt_name = "f16" if fmt == bt.FORMAT_F16 else "bf16"
    if offsets is None:
        exp = O.batch_topk_half(bits, k, seg_len=bits.shape[1], threads=THREADS, fmt=fmt_name)
        plain = run_fixed(bits, k, fmt=fmt_name)
        lengths = np.full(bits.shape[0], bits.shape[1])
    else:
        exp = O.batch_topk_half(bits, k, offsets=offsets.astype(np.int64), threads=THREADS, fmt=fmt_name)
        plain = run_segmented(bits, offsets, k, max_len, fmt=fmt_name)
        lengths = np.diff(offsets)
    ev, ei = exp  # ranks past a segment's length hold the pad, as the entry points write it
    assert_same(plain, (ev, ei), f"{what} plain entry point vs oracle")
    announce(f"ex flags=0 {what}")
    assert_same(run_ex(bits, k, 0, fmt, offsets, max_len), (ev, ei), f"{what} flags=0 vs oracle")

    announce(f"ex indices only {what}")
    v, i = run_ex(bits, k, bt.INDICES_ONLY, fmt, offsets, max_len)
    assert np.array_equal(i, ei), f"{what} indices only vs oracle"
    assert np.all(v == SENTINEL), f"{what}: values written by an indices-only call"

    for flags in (bt.UNSORTED, bt.UNSORTED | bt.INDICES_ONLY):
        announce(f"ex flags={flags} {what}")
        v, i = run_ex(bits, k, flags, fmt, offsets, max_len)
        for r in range(i.shape[0]):
            m = int(min(k, lengths[r]))
            got_i = i[r, :m]
            order = np.argsort(got_i, kind="stable")
            exp_order = np.argsort(ei[r, :m], kind="stable")
            assert np.array_equal(got_i[order], ei[r, :m][exp_order]), (what, flags, r)
            assert np.all(i[r, m:] == -1), (what, flags, r)
            if flags & bt.INDICES_ONLY:
                assert np.all(v[r] == SENTINEL), (what, flags, r)
            else:
                assert np.array_equal(v[r, :m][order], ev[r, :m][exp_order]), (what, flags, r)
                assert np.all(v[r, m:] == 0xFFFF), (what, flags, r)


def _rows(kind, rng, seg_num, seg_len):
    if kind == "normal":
        return rng.standard_normal((seg_num, seg_len)).astype(np.float16).view(np.uint16)
    if kind == "ties":
        return (rng.integers(-4, 5, size=(seg_num, seg_len)) * 0.25).astype(np.float16).view(np.uint16)
    if kind == "specials":
        x = rng.standard_normal((seg_num, seg_len)).astype(np.float16).view(np.uint16)
        n = seg_num * seg_len
        flat = x.reshape(-1)
        flat[rng.integers(0, n, size=n // 20)] = 0x7E00       # NaN
        flat[rng.integers(0, n, size=n // 20)] = 0xFC00       # -inf
        flat[rng.integers(0, n, size=n // 20)] = 0x8000       # -0
        flat[rng.integers(0, n, size=n // 20)] = 0x0000       # +0
        return x
    raise KeyError(kind)


# shapes reaching every selection branch: row ranking (<= 128 candidates), the unsorted
# radix select (longer lists), the pair merge, the three-chunk merge and the cooperative plan
@pytest.mark.parametrize("seg_num,seg_len,k", [
    (16, 4096, 50), (256, 32000, 256), (16, 4096, 200), (5, 300, 300), (8, 200000, 256),
    (4, 300000, 128), (1, 2_000_000, 1024),
])
@pytest.mark.parametrize("kind", ["normal", "ties", "specials"])
def test_ex_fixed_variants(seg_num, seg_len, k, kind):
    rng = np.random.default_rng(seg_num * 7 + seg_len + k)
    bits = _rows(kind, rng, seg_num, seg_len)
    check_variants(bits, k, f"{kind} {seg_num}x{seg_len} k={k}")


def test_ex_segmented_and_bf16_variants():
    rng = np.random.default_rng(5)
    lengths = np.array([0, 1, 63, 64, 65, 300, 5000, 65536, 40000, 7, 0, 131000], dtype=np.int64)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    bits = rng.standard_normal(int(offsets[-1])).astype(np.float16).view(np.uint16)
    for k in (64, 300):
        check_variants(bits, k, f"segmented k={k}", offsets=offsets, max_len=131072)
    f32 = rng.standard_normal((64, 20000)).astype(np.float32)
    bf = (f32.view(np.uint32) >> 16).astype(np.uint16)
    check_variants(bf, 256, "bf16 64x20000 k=256", fmt=bt.FORMAT_BF16)


def test_torch_mirror_sorted_and_values_options():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(9)
    bits = rng.standard_normal((32, 30000)).astype(np.float16)
    x = torch.from_numpy(bits).to("cuda:0")
    announce("torch mirror sorted/values options")
    v, i = bt.topk(x, 200)
    vu, iu = bt.topk(x, 200, sorted=False)
    vn, inn = bt.topk(x, 200, values=False)
    torch.cuda.synchronize()
    ev, ei = O.batch_topk_half(bits.view(np.uint16), 200, seg_len=30000, threads=THREADS)
    assert np.array_equal(i.cpu().numpy(), ei)
    assert np.array_equal(v.view(torch.int16).cpu().numpy().view(np.uint16), ev)
    assert vn is None and torch.equal(inn, i)
    si, order = torch.sort(iu.long(), dim=1)
    se, order_e = torch.sort(i.long(), dim=1)
    assert torch.equal(si, se)
    assert torch.equal(torch.gather(vu, 1, order), torch.gather(v, 1, order_e))
