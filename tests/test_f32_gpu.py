"""GPU parity of the fp32 entry points (radix_topk_batch_topk_f32 / _f32_segmented and the
extended entry point with RADIX_TOPK_FORMAT_F32) against the fp32 oracle: bit-exact indices
and raw 32-bit value patterns (NaN payloads and the sign of zero preserved)."""

import numpy as np
import pytest

import batch_topk_amd as bt
from oracle import oracle as O
from tests.gpu_util import announce, assert_same

pytestmark = pytest.mark.gpu

THREADS = 8
SPECIALS = np.array([0x7FC00000, 0xFFC00001, 0x7F800001, 0x7FFFFFFF, 0x00000000, 0x80000000,
                     0x7F800000, 0xFF800000, 0x00000001, 0x80000001, 0x007FFFFF], dtype=np.uint32)


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    bt.load_library()


def _device_u32(flat, pad_front=0, pad_back=4):
    import torch

    host = np.full(flat.size + pad_front + pad_back, 0x7FC00000, dtype=np.uint32)
    host[pad_front:pad_front + flat.size] = flat
    return torch.from_numpy(host.view(np.int32)).to("cuda:0")


def run_f32(bits, k, offsets=None, max_len=None, elem_offset=0, poison=0xA5, flags=None):
    """fp32 top-k on the GPU -> (values uint32 [S, k], indices int32 [S, k])."""
    import torch

    flat = np.ascontiguousarray(bits, dtype=np.uint32).reshape(-1)
    buf = _device_u32(flat, pad_front=elem_offset)
    in_ptr = buf.data_ptr() + 4 * elem_offset
    if offsets is None:
        seg_num, seg_len = bits.shape
        ws_bytes = bt.batch_topk_f32_workspace_size(seg_num, seg_len, k)
    else:
        seg_num, seg_len = offsets.size - 1, max_len
        ws_bytes = bt.batch_topk_f32_segmented_workspace_size(seg_num, max_len, k)
        d_off = torch.from_numpy(offsets.astype(np.int32)).to("cuda:0")
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
    ws.fill_(poison)
    vals = torch.full((seg_num, k), 0x1234, dtype=torch.int32, device="cuda:0")
    idx = torch.full((seg_num, k), -7, dtype=torch.int32, device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    if flags is not None:
        rc = bt.batch_topk_ex(in_ptr, bt.FORMAT_F32, 0 if offsets is None else d_off.data_ptr(), seg_num,
                              seg_len, k, flags, 0 if flags & bt.INDICES_ONLY else vals.data_ptr(),
                              idx.data_ptr(), ws.data_ptr(), ws_bytes, stream)
    elif offsets is None:
        rc = bt.batch_topk_f32(in_ptr, seg_num, seg_len, k, vals.data_ptr(), idx.data_ptr(),
                               ws.data_ptr(), ws_bytes, stream)
    else:
        rc = bt.batch_topk_f32_segmented(in_ptr, d_off.data_ptr(), seg_num, max_len, k, vals.data_ptr(),
                                         idx.data_ptr(), ws.data_ptr(), ws_bytes, stream)
    assert rc == 0
    torch.cuda.synchronize()
    return vals.cpu().numpy().view(np.uint32), idx.cpu().numpy()


def check(bits, k, what, offsets=None, max_len=None, elem_offset=0):
    announce(f"f32 {what} k={k} offset={elem_offset}")
    got = run_f32(bits, k, offsets=offsets, max_len=max_len, elem_offset=elem_offset)
    if offsets is None:
        exp = O.batch_topk_half(bits, k, seg_len=bits.shape[1], threads=THREADS, fmt="f32")
    else:
        exp = O.batch_topk_half(bits, k, offsets=offsets.astype(np.int64), threads=THREADS, fmt="f32")
    assert_same(got, exp, f"f32 {what}")
    return got


def _bits(kind, rng, n):
    if kind == 0:
        return rng.standard_normal(n).astype(np.float32).view(np.uint32)
    if kind == 1:   # heavy ties
        return (rng.integers(-8, 9, size=n) * 0.5).astype(np.float32).view(np.uint32)
    if kind == 2:   # sorted
        return np.sort(rng.standard_normal(n).astype(np.float32)).view(np.uint32)
    if kind == 3:   # specials sprinkled
        b = rng.standard_normal(n).astype(np.float32).view(np.uint32).copy()
        pos = rng.integers(0, n, size=max(1, n // 20))
        b[pos] = SPECIALS[rng.integers(0, SPECIALS.size, size=pos.size)]
        return b
    if kind == 4:   # values that differ only below the 16-bit key prefix
        return (np.float32(3.0) + rng.integers(0, 4096, size=n).astype(np.float32) * np.float32(2 ** -22)).view(np.uint32)
    return rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)   # any pattern


def test_f32_reference_kats():
    f = lambda v: np.asarray(v, dtype=np.float32).view(np.uint32)
    v, i = run_f32(f([[5, 7, 7, 1]]), 2)
    assert i[0].tolist() == [1, 2] and v[0].view(np.float32).tolist() == [7, 7]
    v, i = run_f32(f([[np.nan, 3, -1, np.nan]]), 3)
    assert i[0].tolist() == [1, 2, 0]
    v, i = run_f32(f([2, 1]), 4, offsets=np.array([0, 2]), max_len=4)
    assert i[0].tolist() == [0, 1, -1, -1] and v[0][2:].tolist() == [0xFFFFFFFF] * 2


@pytest.mark.parametrize("case", range(24))
def test_f32_random_fixed_shapes(case):
    rng = np.random.default_rng(5000 + case)
    seg_len = int(rng.choice([1, 7, 100, 1000, 4096, 9999, 33000, 70000, 131072, 200000, 400001]))
    seg_num = int(rng.integers(1, max(2, min(600, 3_000_000 // seg_len))))
    k = int(min(seg_len, rng.choice([1, 2, 17, 50, 64, 100, 128, 200, 256, 513, 1024])))
    bits = _bits(int(rng.integers(0, 6)), rng, seg_num * seg_len).reshape(seg_num, seg_len)
    check(bits, k, f"random fixed case {case} {seg_num}x{seg_len}", elem_offset=int(rng.integers(0, 4)))


@pytest.mark.parametrize("case", range(8))
def test_f32_random_segmented_shapes(case):
    rng = np.random.default_rng(6000 + case)
    seg_num = int(rng.integers(1, 600))
    max_len = int(rng.choice([10, 1000, 65536, 131072, 300000]))
    lengths = rng.integers(0, max_len + 1, size=seg_num).astype(np.int64)
    while lengths.sum() > 6_000_000:
        lengths //= 2
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    k = int(rng.choice([1, 16, 64, 128, 256]))
    bits = _bits(int(rng.integers(0, 6)), rng, int(offsets[-1]))
    check(bits, k, f"random segmented case {case}", offsets=offsets, max_len=max_len,
          elem_offset=int(rng.integers(0, 4)))


# one row per plan branch: single chunk, two chunks (pair merge), three chunks (last-arriver
# merge), cooperative; special rows on each
@pytest.mark.parametrize("seg_num,seg_len,k", [
    (128, 32000, 50), (64, 100000, 50), (4, 150000, 64), (1, 4_000_000, 1024), (3, 250000, 512),
])
def test_f32_plan_branches_with_special_rows(seg_num, seg_len, k):
    rng = np.random.default_rng(seg_len + k)
    bits = rng.standard_normal((seg_num, seg_len)).astype(np.float32).view(np.uint32).copy()
    if seg_num >= 3:
        bits[0] = 0x80000000                                            # all -0
        bits[1] = SPECIALS[rng.integers(0, SPECIALS.size, size=seg_len)]
        bits[2, ::3] = 0x7FC00000 | rng.integers(0, 2**22, size=bits[2, ::3].size).astype(np.uint32)
    check(bits, k, f"plan branch {seg_num}x{seg_len}", elem_offset=1)


def _f32_kind(kind, rng, n):
    if kind == "ties":  # 13 distinct values
        x = (rng.integers(-6, 7, size=n) * 0.25).astype(np.float32)
    elif kind == "sorted":  # every top value in the last chunk
        x = np.sort(rng.standard_normal(n).astype(np.float32))
    elif kind == "descending":  # every top value in the first chunk
        x = -np.sort(rng.standard_normal(n).astype(np.float32))
    elif kind == "nan_inf":  # NaNs with random payloads, -inf and a few +inf among normals
        x = rng.standard_normal(n).astype(np.float32)
        r = rng.random(n)
        x[r < 0.3] = np.nan
        x[(r >= 0.3) & (r < 0.5)] = -np.inf
        x[r > 0.99995] = np.inf
    else:
        raise KeyError(kind)
    bits = x.view(np.uint32).copy()
    if kind == "nan_inf":
        nan = np.isnan(x)
        bits[nan] = 0x7F800001 | rng.integers(0, 2**22, size=int(nan.sum())).astype(np.uint32)
    return bits


# the cooperative path (segments over many co-resident workgroups) on tied, ordered and
# NaN-heavy fp32 rows: 32-bit keys take up to 8 refinement digits when the lists overflow
@pytest.mark.parametrize("seg_num,seg_len,k,kind", [
    (1, 1_000_000, 1024, "ties"), (1, 1_000_000, 1024, "sorted"), (1, 1_000_000, 1024, "descending"),
    (1, 1_000_000, 1024, "nan_inf"), (2, 3_000_000, 64, "ties"), (2, 3_000_000, 64, "sorted"),
])
def test_f32_cooperative_data_kinds(seg_num, seg_len, k, kind):
    rng = np.random.default_rng(seg_len + k)
    bits = _f32_kind(kind, rng, seg_num * seg_len).reshape(seg_num, seg_len)
    check(bits, k, f"cooperative {kind} {seg_num}x{seg_len}")


def test_f32_ex_flags_and_torch_mirror():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(21)
    bits = _bits(3, rng, 64 * 20000).reshape(64, 20000)
    plain = O.batch_topk_half(bits, 256, seg_len=20000, threads=THREADS, fmt="f32")
    assert_same(run_f32(bits, 256), plain, "f32 plain entry point vs oracle")
    announce("f32 ex flags")
    assert_same(run_f32(bits, 256, flags=0), plain, "f32 ex flags=0 vs oracle")
    v, i = run_f32(bits, 256, flags=bt.UNSORTED)
    for r in range(64):
        o, e = np.argsort(i[r]), np.argsort(plain[1][r])
        assert np.array_equal(i[r][o], plain[1][r][e]) and np.array_equal(v[r][o], plain[0][r][e])
    v, i = run_f32(bits, 256, flags=bt.INDICES_ONLY)
    assert np.array_equal(i, plain[1]) and np.all(v == 0x1234)
    x = torch.from_numpy(bits.view(np.float32)).to("cuda:0")
    tv, ti = bt.topk(x, 256)
    torch.cuda.synchronize()
    assert np.array_equal(ti.cpu().numpy(), plain[1])
    assert np.array_equal(tv.cpu().numpy().view(np.uint32), plain[0])


def test_f32_huge_segment_uses_every_cu_when_aligned():
    # 2^24 floats, k = 1024: 256 cooperative chunks of 65,536 when the row is 16-byte aligned
    # (the plan reserves a 257th for misalignment; the launch uses the exact count)
    import torch

    rng = np.random.default_rng(77)
    n = 1 << 24
    bits = rng.standard_normal(n).astype(np.float32).view(np.uint32).reshape(1, n)
    check(bits, 1024, "1 x 2^24 aligned")
    # the same row one element off alignment needs 257 co-resident workgroups: refused at
    # launch with hipErrorCooperativeLaunchTooLarge (720), nothing is launched
    announce("f32 1 x 2^24 misaligned: refused")
    buf = _device_u32(bits.reshape(-1), pad_front=1)
    ws_bytes = bt.batch_topk_f32_workspace_size(1, n, 1024)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
    vals = torch.empty((1, 1024), dtype=torch.int32, device="cuda:0")
    idx = torch.empty((1, 1024), dtype=torch.int32, device="cuda:0")
    rc = bt.batch_topk_f32(buf.data_ptr() + 4, 1, n, 1024, vals.data_ptr(), idx.data_ptr(),
                           ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    assert rc == 720


# the many-row plan (at least 512 rows): 256-thread workgroups for rows of at most 4,096
# floats, and of at most 8,192 (8 vectors per thread) from 768 rows on; 512 threads otherwise
# (700 x 4,097 and 600 x 8,193 here); misaligned starts give some rows a tail workgroup
@pytest.mark.parametrize("seg_num,seg_len,k,kind", [
    (2000, 2000, 50, None), (4096, 1024, 64, "ties"), (1000, 4096, 50, "nan_inf"),
    (700, 4097, 50, None), (600, 4096, 1, "sorted"), (512, 3000, 128, "descending"),
    (1000, 8192, 64, "ties"), (600, 8193, 50, None),
])
def test_f32_many_row_plan(seg_num, seg_len, k, kind):
    rng = np.random.default_rng(seg_num + seg_len + k)
    n = seg_num * seg_len
    bits = (rng.standard_normal(n).astype(np.float32).view(np.uint32) if kind is None
            else _f32_kind(kind, rng, n)).reshape(seg_num, seg_len)
    check(bits, k, f"many-row plan {seg_num}x{seg_len} {kind}", elem_offset=3)


@pytest.mark.parametrize("seg_num,max_len,k", [(1000, 4096, 50), (3000, 2048, 16), (800, 5000, 64)])
def test_f32_many_row_segmented(seg_num, max_len, k):
    rng = np.random.default_rng(seg_num * 7 + max_len)
    lengths = rng.integers(0, max_len + 1, size=seg_num).astype(np.int64)
    lengths[:4] = [0, 1, max_len, k]
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    bits = rng.standard_normal(int(offsets[-1])).astype(np.float32).view(np.uint32)
    check(bits, k, f"many-row segmented {seg_num} x U[0,{max_len}]", offsets=offsets, max_len=max_len,
          elem_offset=1)
