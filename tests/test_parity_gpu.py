"""GPU parity: the HIP engine, called through the C ABI, against the oracle and the reference
tests' known answers.  Bit-exact on indices and on the raw 16-bit patterns (fp16 or bf16) of every value."""

import json
import os

import numpy as np
import pytest

import batch_topk_amd as bt
from batch_topk_amd import workloads as wl
from oracle import oracle as O
from tests.gpu_util import announce, assert_properties, assert_same, run_fixed, run_segmented

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "kats.json")
THREADS = 8


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    bt.load_library()


def oracle_fixed(bits, k):
    return O.batch_topk_half(bits, k, seg_len=bits.shape[1], threads=THREADS)


def check_fixed(bits, k, what, **kw):
    announce(f"{what} shape={bits.shape} k={k} {kw}")
    got = run_fixed(bits, k, **kw)
    assert_same(got, oracle_fixed(bits, k), what)
    return got


# ------------------------------------------------------------------ reference known answers

def test_golden_cases():
    with open(GOLDEN) as f:
        cases = json.load(f)["cases"]
    for c in cases:
        bits = np.array(c["input_bits"], dtype=np.uint16).reshape(c["seg_num"], c["seg_len"])
        poison = 0xA5 if "poisoned" in c["name"] else None
        announce(f"golden {c['name']}")
        vals, idx = run_fixed(bits, c["k"], poison=poison)
        assert idx.tolist() == c["expected_idx"], c["name"]
        assert vals.tolist() == c["expected_val_bits"], c["name"]


@pytest.mark.parametrize("seg_num,seg_len,k,seed", [
    (1, 10000, 50, 7), (8, 10000, 50, 17), (32, 10000, 50, 23),   # test:596-600
    (3, 256, 128, 2026),                                           # test:817-920
    (128, 10000, 50, 1234),                                        # test:1028-1141
])
def test_reference_random_cases(seg_num, seg_len, k, seed):
    _, bits = O.make_random_input(seg_num, seg_len, seed)
    check_fixed(bits.reshape(seg_num, seg_len), k, f"reference random seed={seed}")


def test_reference_smoke_all_zero_row():
    # test/test_batch_topk.cu:1319-1385: a zero row of 10000, k = 50 -> indices 0..49.
    bits = np.zeros((1, 10000), dtype=np.uint16)
    vals, idx = check_fixed(bits, 50, "all-zero row")
    assert idx[0].tolist() == list(range(50))


# ------------------------------------------------------------------ the five workloads

def test_uniform_small():
    check_fixed(wl.uniform_small(), 50, "uniform_small 16x4096")


def test_llm_logits_full():
    bits = wl.llm_logits()
    vals, idx = check_fixed(bits, 50, "llm_logits 128x128256")
    assert_properties(bits, vals, idx, 50, [bits.shape[1]] * bits.shape[0])


def test_varlen_segments():
    bits, offsets = wl.varlen()
    announce("varlen 512 segments k=64")
    got = run_segmented(bits, offsets, 64, 65536, poison=0xA5)
    exp = O.batch_topk_half(bits, 64, offsets=offsets.astype(np.int64), threads=THREADS)
    assert_same(got, exp, "varlen")
    lengths = np.diff(offsets)
    assert np.all(got[1][lengths == 1, 1:] == bt.PAD_INDEX)


@pytest.mark.parametrize("k", [1, 16, 128, 256])
def test_ties_special(k):
    bits = wl.ties_special()
    check_fixed(bits, k, "ties_special 256x32000")


def test_huge_segment():
    if bt.batch_topk_half_workspace_size(1, 16_777_216, 1024) == 0:
        pytest.skip("single-segment path for 16,777,216 elements with k = 1024 not built yet")
    bits = wl.huge_segment()
    check_fixed(bits, 1024, "huge_segment 1x16777216")


# ------------------------------------------------------------------ edge cases

def _edge_rows():
    rng = np.random.default_rng(99)
    rows = {}
    rows["all_equal"] = np.full((3, 5000), 0x3C00, dtype=np.uint16)
    rows["all_nan"] = np.tile(np.array([0x7E00, 0xFE00, 0x7C01, 0xFFFF], dtype=np.uint16), (2, 1250))
    rows["all_neg_inf"] = np.full((2, 3000), 0xFC00, dtype=np.uint16)
    rows["all_negative"] = (rng.integers(0x8001, 0xFBFF, size=(4, 7000))).astype(np.uint16)
    rows["signed_zeros"] = rng.choice(np.array([0x0000, 0x8000], dtype=np.uint16), size=(2, 4000))
    x = rng.integers(0, 65536, size=(4, 9001)).astype(np.uint16)
    rows["random_bits"] = x
    y = np.full((2, 6000), 0xBC00, dtype=np.uint16)
    y[:, rng.integers(0, 6000, size=100)] = 0x7E00
    rows["nan_sprinkled_negatives"] = y
    z = np.sort(rng.standard_normal((2, 20000)).astype(np.float16), axis=1).view(np.uint16)
    rows["sorted_ascending"] = z
    rows["sorted_descending"] = z[:, ::-1].copy()
    d = (rng.integers(-3, 4, size=(2, 40000)) * 0.5).astype(np.float16).view(np.uint16)
    rows["few_distinct_long"] = d
    rows["subnormals"] = rng.integers(0x0001, 0x03FF, size=(2, 5000)).astype(np.uint16) | \
        (rng.integers(0, 2, size=(2, 5000)).astype(np.uint16) << 15)
    return rows


@pytest.mark.parametrize("name", list(_edge_rows().keys()))
@pytest.mark.parametrize("k", [1, 50, 300])
def test_edge_rows(name, k):
    bits = _edge_rows()[name]
    if k > bits.shape[1]:
        pytest.skip("k > seg_len")
    vals, idx = check_fixed(bits, k, f"edge {name}")
    assert_properties(bits, vals, idx, k, [bits.shape[1]] * bits.shape[0])


@pytest.mark.parametrize("seg_len", [4096, 32000, 128256])
@pytest.mark.parametrize("k", [1, 50])
def test_top_values_next_to_positive_nans(seg_len, k):
    # Every top element shares its 16-byte vector with a positive NaN (0x7E00 / 0x7C01 /
    # 0x7FFF), so the raw int16 maximum of every lane holding a top element is a NaN.  Those
    # lanes must still be searched for candidates (a NaN is the worst value, never selected
    # ahead of a real one).
    rng = np.random.default_rng(seg_len + k)
    bits = rng.standard_normal((4, seg_len)).astype(np.float16).view(np.uint16)
    nans = np.array([0x7E00, 0x7C01, 0x7FFF], dtype=np.uint16)
    for r in range(bits.shape[0]):
        top = rng.choice(seg_len, size=60, replace=False)
        bits[r, top] = (np.float16(40.0) + rng.integers(0, 8, size=60).astype(np.float16)).view(np.uint16)
        bits[r, top ^ 1] = nans[rng.integers(0, 3, size=60)]
    check_fixed(bits, k, f"top values beside positive NaNs seg_len={seg_len}")


@pytest.mark.parametrize("seg_len,k", [(1, 1), (7, 7), (8, 3), (63, 63), (64, 50), (65, 64),
                                       (257, 256), (1000, 1000), (4096, 1024), (4097, 1)])
def test_small_and_k_equal_len(seg_len, k):
    rng = np.random.default_rng(seg_len * 31 + k)
    bits = rng.standard_normal((5, seg_len)).astype(np.float16).view(np.uint16)
    check_fixed(bits, k, f"small seg_len={seg_len}")


@pytest.mark.parametrize("elem_offset", [1, 3, 7])
@pytest.mark.parametrize("seg_len", [4099, 40001])
def test_misaligned_input(elem_offset, seg_len):
    rng = np.random.default_rng(elem_offset)
    bits = rng.standard_normal((6, seg_len)).astype(np.float16).view(np.uint16)
    check_fixed(bits, 50, "misaligned", elem_offset=elem_offset)


def test_multichunk_ties_across_chunks():
    # equal values spread across several workgroups of one segment: index order must hold
    bits = np.full((4, 100_000), 0x3C00, dtype=np.uint16)
    bits[:, ::997] = 0x4000
    for k in (1, 50, 150, 700):
        check_fixed(bits, k, "multichunk ties")


def test_repeated_calls_share_workspace():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    a = rng.standard_normal((16, 60000)).astype(np.float16).view(np.uint16)
    ws = torch.empty(bt.batch_topk_half_workspace_size(16, 60000, 50), dtype=torch.uint8,
                     device="cuda:0")
    ws.fill_(0xA5)
    for rep in range(3):
        announce(f"repeated call {rep}")
        got = run_fixed(a, 50, workspace=ws)
        assert_same(got, oracle_fixed(a, 50), f"repeat {rep}")


def test_varlen_edge_segments():
    rng = np.random.default_rng(17)
    lengths = np.array([0, 1, 2, 7, 8, 9, 63, 64, 65, 1000, 0, 65536, 33333, 5, 0], dtype=np.int64)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    bits = rng.standard_normal(int(offsets[-1])).astype(np.float16).view(np.uint16)
    for k, elem_offset in ((64, 0), (64, 3), (1, 5), (200, 0)):
        announce(f"varlen edges k={k} offset={elem_offset}")
        got = run_segmented(bits, offsets, k, 65536, elem_offset=elem_offset)
        exp = O.batch_topk_half(bits, k, offsets=offsets.astype(np.int64), threads=THREADS)
        assert_same(got, exp, f"varlen edges k={k}")


def test_varlen_segment_longer_than_declared_max_is_padded():
    rng = np.random.default_rng(2)
    lengths = np.array([100, 5000, 100], dtype=np.int64)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    bits = rng.standard_normal(int(offsets[-1])).astype(np.float16).view(np.uint16)
    announce("varlen precondition violation")
    vals, idx = run_segmented(bits, offsets, 10, 200)
    exp = O.batch_topk_half(bits, 10, offsets=offsets.astype(np.int64))
    assert np.array_equal(idx[0], exp[1][0]) and np.array_equal(idx[2], exp[1][2])
    assert np.all(idx[1] == -1) and np.all(vals[1] == 0xFFFF)


# ------------------------------------------------------------------ cooperative path
# Segments longer than one workgroup's chunk with k too large for the LDS merge of per-chunk
# lists: every workgroup of the segment shares one threshold from global histograms.

def _coop_rows(name, n):
    rng = np.random.default_rng(len(name) * 7 + n % 97)
    if name == "normal":
        return rng.standard_normal((1, n)).astype(np.float16).view(np.uint16)
    if name == "all_equal":
        return np.full((1, n), 0x3C00, dtype=np.uint16)
    if name == "all_nan":
        return np.tile(np.array([0x7E00, 0xFE00, 0x7C01, 0xFFFF], dtype=np.uint16), (1, n // 4))
    if name == "sorted_ascending":
        return np.sort(rng.standard_normal((1, n)).astype(np.float16), axis=1).view(np.uint16)
    if name == "sorted_descending":
        return np.sort(rng.standard_normal((1, n)).astype(np.float16), axis=1)[:, ::-1].copy().view(np.uint16)
    if name == "few_distinct":
        return (rng.integers(-4, 5, size=(1, n)) * 0.25).astype(np.float16).view(np.uint16)
    raise KeyError(name)


@pytest.mark.parametrize("name", ["normal", "all_equal", "all_nan", "sorted_ascending",
                                  "sorted_descending", "few_distinct"])
def test_cooperative_single_segment(name):
    bits = _coop_rows(name, 1_000_000)
    for k in (300, 1024):
        vals, idx = check_fixed(bits, k, f"cooperative {name}")
        assert_properties(bits, vals, idx, k, [bits.shape[1]])


def test_cooperative_several_segments():
    rng = np.random.default_rng(31)
    bits = rng.standard_normal((3, 300_001)).astype(np.float16).view(np.uint16)
    bits[1, 1000:200000] = 0x4400  # a long run of equal large values in one segment
    check_fixed(bits, 512, "cooperative 3 segments", elem_offset=3)


def test_cooperative_variable_segments():
    rng = np.random.default_rng(37)
    lengths = np.array([400_000, 5, 0, 300_000, 150_000, 131_072, 131_073], dtype=np.int64)
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    bits = rng.standard_normal(int(offsets[-1])).astype(np.float16).view(np.uint16)
    bits[offsets[3]:offsets[3] + 50_000] = 0x3C00
    announce("cooperative variable-length segments k=300")
    got = run_segmented(bits, offsets, 300, 400_000, poison=0x5A)
    exp = O.batch_topk_half(bits, 300, offsets=offsets.astype(np.int64), threads=THREADS)
    assert_same(got, exp, "cooperative varlen")


# ------------------------------------------------------------------ the reference's benchmark matrix

@pytest.mark.parametrize("seg_num", [128, 1500, 6000])
def test_reference_benchmark_matrix(seg_num):
    # bench/bench_batch_topk.cu:9-15 fill pattern at the shapes of
    # include/batch_topk_benchmark.cuh:14-20 (heavy ties: 2048 distinct values per period)
    bits = wl.ref_matrix(seg_num)
    check_fixed(bits, 50, f"reference bench matrix {seg_num}x10000")


# ------------------------------------------------------------------ many segments, tail chunks
# With at least two segments per CU the plan takes the smallest workgroup covering max_len;
# a segment whose misaligned span reaches past that chunk gets a second (tail) workgroup.

def test_many_segments_with_tail_chunks():
    rng = np.random.default_rng(41)
    lengths = rng.integers(1, 300, size=600).astype(np.int64)
    lengths[[3, 100, 333, 599]] = [65536, 65533, 65530, 65536]
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    bits = rng.standard_normal(int(offsets[-1])).astype(np.float16).view(np.uint16)
    for k, elem_offset in ((64, 3), (1, 7), (64, 0)):
        announce(f"many segments with tail chunks k={k} offset={elem_offset}")
        got = run_segmented(bits, offsets, k, 65536, elem_offset=elem_offset, poison=0x3C)
        exp = O.batch_topk_half(bits, k, offsets=offsets.astype(np.int64), threads=THREADS)
        assert_same(got, exp, f"tail chunks k={k}")


def test_fixed_length_tail_chunks():
    rng = np.random.default_rng(43)
    bits = rng.standard_normal((512, 16384)).astype(np.float16).view(np.uint16)
    check_fixed(bits, 50, "512x16384 misaligned", elem_offset=3)


# ------------------------------------------------------------------ seeded random shapes
# Shape, k, distribution, alignment and entry point drawn from a fixed seed: every plan
# branch (block/vector shapes, tail chunks, multi-chunk merge, cooperative) meets random data.

def _random_bits(rng, n):
    kind = rng.integers(0, 6)
    if kind == 0:
        x = rng.standard_normal(n).astype(np.float16)
    elif kind == 1:
        x = (rng.integers(-8, 9, size=n) * 0.5).astype(np.float16)      # heavy ties
    elif kind == 2:
        x = rng.uniform(-1, 1, size=n).astype(np.float16)
    elif kind == 3:
        x = np.sort(rng.standard_normal(n)).astype(np.float16)          # sorted
    elif kind == 4:
        x = rng.standard_normal(n).astype(np.float16)
        x[rng.integers(0, n, size=max(1, n // 50))] = np.float16(np.inf)
        x[rng.integers(0, n, size=max(1, n // 50))] = np.float16(-np.inf)
    else:
        return rng.integers(0, 65536, size=n).astype(np.uint16)         # any bit pattern
    return x.view(np.uint16)


@pytest.mark.parametrize("case", range(24))
def test_random_fixed_shapes(case):
    rng = np.random.default_rng(1000 + case)
    seg_len = int(rng.choice([1, 7, 100, 1000, 4096, 9999, 33000, 70000, 131072, 200000, 400001]))
    seg_num = int(rng.integers(1, max(2, min(600, 3_000_000 // seg_len))))
    k = int(min(seg_len, rng.choice([1, 2, 17, 50, 64, 100, 128, 200, 256, 513, 1024])))
    bits = _random_bits(rng, seg_num * seg_len).reshape(seg_num, seg_len)
    elem_offset = int(rng.integers(0, 8))
    check_fixed(bits, k, f"random fixed case {case}", elem_offset=elem_offset)


@pytest.mark.parametrize("case", range(12))
def test_random_segmented_shapes(case):
    rng = np.random.default_rng(2000 + case)
    seg_num = int(rng.integers(1, 700))
    max_len = int(rng.choice([10, 1000, 65536, 131072, 300000]))
    lengths = rng.integers(0, max_len + 1, size=seg_num).astype(np.int64)
    while lengths.sum() > 6_000_000:
        lengths //= 2
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    k = int(rng.choice([1, 16, 50, 64, 128, 300, 1024]))
    if bt.batch_topk_half_segmented_workspace_size(seg_num, max_len, k) == 0:
        # beyond the cooperative grid limit (segments x chunks > 256 workgroups)
        pytest.skip(f"unsupported shape seg_num={seg_num} max_len={max_len} k={k}")
    bits = _random_bits(rng, max(1, int(offsets[-1])))
    elem_offset = int(rng.integers(0, 8))
    announce(f"random segmented case {case}: seg_num={seg_num} max_len={max_len} k={k}")
    got = run_segmented(bits, offsets, k, max_len, elem_offset=elem_offset, poison=0x77)
    exp = O.batch_topk_half(bits, k, offsets=offsets.astype(np.int64), threads=THREADS)
    assert_same(got, exp, f"random segmented case {case}")


# ------------------------------------------------------------------ bfloat16 entry points

BF16_SPECIALS = np.array([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0xFFC1, 0x7F81, 0x3F80, 0xBF80],
                         dtype=np.uint16)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    torch = pytest.importorskip("torch")
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).bfloat16().view(torch.int16) \
        .numpy().view(np.uint16)


def check_bf16(bits, k, what, **kw):
    announce(f"bf16 {what} shape={bits.shape} k={k} {kw}")
    got = run_fixed(bits, k, fmt="bf16", **kw)
    exp = O.batch_topk_half(bits, k, seg_len=bits.shape[1], threads=THREADS, fmt="bf16")
    assert_same(got, exp, f"bf16 {what}")
    return got


@pytest.mark.parametrize("seg_num,seg_len,k", [
    (16, 4096, 50), (3, 257, 256), (5, 9001, 1), (8, 32000, 128), (4, 131072, 64),
    (3, 300_000, 50), (2, 200_000, 300), (1, 1_000_000, 1024),
])
def test_bf16_random_with_specials(seg_num, seg_len, k):
    rng = np.random.default_rng(seg_len + k)
    bits = to_bf16_bits(rng.standard_normal((seg_num, seg_len)) * 3.0)
    mask = rng.random(bits.shape) < 0.01
    bits[mask] = BF16_SPECIALS[rng.integers(0, BF16_SPECIALS.size, size=int(mask.sum()))]
    vals, idx = check_bf16(bits, k, "random with specials")
    assert_properties(bits, vals, idx, k, [seg_len] * seg_num, fmt="bf16")


def test_bf16_llm_logits_full():
    # The LLM-logits rows (128 x 128,256, N(0, sd 2) with a +8 boosted tail) rounded to bfloat16.
    bits = to_bf16_bits(wl.llm_logits().view(np.float16).astype(np.float32))
    vals, idx = check_bf16(bits, 50, "llm_logits")
    assert_properties(bits, vals, idx, 50, [bits.shape[1]] * bits.shape[0], fmt="bf16")


@pytest.mark.parametrize("k", [1, 16, 256])
def test_bf16_ties_and_specials(k):
    # 64 distinct values, 1 % -inf, 0.5 % NaN of every encoding, +-0: bit-exact tie order.
    rng = np.random.default_rng(k)
    table = to_bf16_bits((np.arange(64) - 32) / 8.0)
    bits = table[rng.integers(0, 64, size=(32, 20000))]
    bits[rng.random(bits.shape) < 0.01] = 0xFF80
    nan_mask = rng.random(bits.shape) < 0.005
    bits[nan_mask] = np.array([0x7FC0, 0xFFC1, 0x7F81, 0xFFFF], dtype=np.uint16)[
        rng.integers(0, 4, size=int(nan_mask.sum()))]
    check_bf16(bits, k, "ties and specials")


def test_bf16_top_values_next_to_positive_nans():
    rng = np.random.default_rng(5)
    bits = to_bf16_bits(rng.standard_normal((4, 40000)))
    for r in range(4):
        top = rng.choice(40000, size=60, replace=False)
        bits[r, top] = to_bf16_bits(40.0 + rng.integers(0, 8, size=60))
        bits[r, top ^ 1] = np.array([0x7FC0, 0x7F81, 0x7FFF], dtype=np.uint16)[rng.integers(0, 3, size=60)]
    check_bf16(bits, 50, "top values beside positive NaNs")


def test_bf16_segmented():
    rng = np.random.default_rng(21)
    lengths = rng.integers(0, 70000, size=40)
    lengths[:6] = [0, 1, 7, 49, 64, 65]
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    bits = to_bf16_bits(rng.standard_normal(int(offsets[-1])))
    announce("bf16 segmented 40 segments k=64")
    got = run_segmented(bits, offsets, 64, 70000, fmt="bf16")
    exp = O.batch_topk_half(bits, 64, offsets=offsets, threads=THREADS, fmt="bf16")
    assert_same(got, exp, "bf16 segmented")


def test_bf16_torch_convenience():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    bits = to_bf16_bits(rng.standard_normal((6, 5000)))
    x = torch.from_numpy(bits.view(np.int16)).to("cuda:0").view(torch.bfloat16)
    announce("bf16 torch topk 6x5000 k=20")
    vals, idx = bt.topk(x, 20)
    torch.cuda.synchronize()
    ev, ei = O.batch_topk_half(bits, 20, seg_len=5000, fmt="bf16")
    assert vals.dtype == torch.bfloat16
    assert np.array_equal(idx.cpu().numpy(), ei)
    assert np.array_equal(vals.view(torch.int16).cpu().numpy().view(np.uint16), ev)


# Lists of 256 to 512 candidates are ranked by sorted runs: on u32 keys (key16 << 16 | index16)
# in 16-bit rows shorter than 65,535 elements, on the u64 candidates otherwise.  Both sides of
# that bound, fp16 and bf16, on rows of 512 distinct values (about 128 copies of each, so the
# threshold's ties make lists of 350-400), with NaNs and -inf at the last positions.
@pytest.mark.parametrize("seg_len", [65533, 65534, 65535, 65536])
@pytest.mark.parametrize("fmt", ["f16", "bf16"])
def test_sorted_runs_index_bound(seg_len, fmt):
    rng = np.random.default_rng(seg_len)
    v = (rng.integers(0, 512, size=(3, seg_len)) - 256) / 64.0
    if fmt == "f16":
        bits = v.astype(np.float16).view(np.uint16)
        nan, ninf = 0x7E00, 0xFC00
    else:
        bits = to_bf16_bits(v)
        nan, ninf = 0x7FC0, 0xFF80
    bits[:, -1] = nan
    bits[:, -2] = ninf
    bits[1, -3] = nan | 0x8000
    what = f"sorted runs at the index bound {seg_len} {fmt}"
    announce(f"{what} k=300")
    got = run_fixed(bits, 300, fmt=fmt)
    exp = O.batch_topk_half(bits, 300, seg_len=seg_len, threads=THREADS, fmt=fmt)
    assert_same(got, exp, what)
