"""Pins the oracle (oracle/oracle.cpp + oracle/oracle.py) before it is trusted as the checker.

Each check compares the oracle with something other than itself: the reference tests'
known answers (tests/golden/kats.json, derived from closed forms), numpy's IEEE-754
float16 implementation, an independent numpy statement of the order, and brute force.
"""

import itertools
import json
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "kats.json")


@pytest.fixture(scope="module")
def kats():
    with open(GOLDEN) as f:
        return json.load(f)


# ------------------------------------------------------------------ codec and conversions

def test_codec_known_answers(kats):
    # test/test_batch_topk.cu:46-51 plus the closed-form table of include/type_codec.cuh
    for bits, key in kats["codec_desc"]:
        assert O.encode_half_desc(bits) == key, hex(bits)
    neg = O.encode_half_desc(0xBC00)   # -1
    pos = O.encode_half_desc(0x4200)   # 3
    nan = O.encode_half_desc(0x7E00)
    assert pos < neg and nan > neg


def test_codec_exhaustive_monotone_against_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    keys = np.array([O.encode_half_desc(int(b)) for b in bits], dtype=np.int64)
    np.testing.assert_array_equal(keys, O.encode_half_desc_np(bits).astype(np.int64))
    f = bits.view(np.float16).astype(np.float64)
    nan = np.isnan(f)
    assert np.all(keys[nan] == 0xFFFF)
    # strictly decreasing in value, equal keys exactly for equal values (+0 == -0)
    fin = ~nan
    fv, kv = f[fin], keys[fin]
    order = np.argsort(-fv, kind="stable")
    fs, ks = fv[order], kv[order]
    assert np.all(np.diff(ks) >= 0)
    assert np.all((np.diff(ks) == 0) == (np.diff(fs) == 0))
    assert keys[0x0000] == keys[0x8000] == 0x7FFF
    assert O.encode_half_asc(0x7C00) == 0xFC00 and O.normalize_half_bits(0xFC01) == 0xFFFF


def test_half_to_float_matches_numpy_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    got = O.half_to_float(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_matches_numpy_rne():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32) * np.float32(1e-5),   # subnormals
        rng.standard_normal(200_000).astype(np.float32) * np.float32(300),
        rng.uniform(-70000, 70000, 50_000).astype(np.float32),                 # overflow
        O.half_to_float(np.arange(0, 0x7C00, dtype=np.uint16)),                 # exact halves
        (np.arange(0, 0x7BFF, dtype=np.float32) + 0.5),                         # ties
    ])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(O.float_to_half(x), ref)


def test_candidate_better_tie_break():
    # test/test_batch_topk.cu:53-64
    five = 0x4500
    assert not O.candidate_better(five, 2, five, 1)
    assert O.candidate_better(five, 1, five, 2)
    assert O.candidate_better(0xBC00, 9, 0x7E00, 0)       # -1 beats NaN
    assert not O.candidate_better(0x0000, 3, 0x8000, 2)   # +0 == -0, index decides


# ------------------------------------------------------------------ cpu_reference_topk

def test_reference_host_kats():
    # test/test_batch_topk.cu:19-44
    v, i = O.cpu_reference_topk([5, 7, 7, 1], 4, 2)
    assert i == [1, 2] and v == [7, 7]
    v, i = O.cpu_reference_topk([np.nan, 3, -1, np.nan], 4, 3)
    assert i == [1, 2, 0] and v[:2] == [3, -1] and np.isnan(v[2])
    v, i = O.cpu_reference_topk([2, 1], 4, 4)
    assert i == [0, 1] and v == [2, 1]
    assert O.cpu_reference_topk([1, 2], 0, 3) == ([], [])
    assert O.cpu_reference_topk([1, 2], 2, 0) == ([], [])


def test_golden_cases(kats):
    for c in kats["cases"]:
        bits = np.array(c["input_bits"], dtype=np.uint16)
        vals, idx = O.batch_topk_half(bits, c["k"], seg_len=c["seg_len"])
        assert idx.tolist() == c["expected_idx"], c["name"]
        assert vals.tolist() == c["expected_val_bits"], c["name"]


SPECIALS = np.array([0x0000, 0x8000, 0x7C00, 0xFC00, 0x7E00, 0xFE00, 0x7C01, 0x3C00, 0xBC00,
                     0x0001, 0x8001, 0x7BFF, 0xFBFF], dtype=np.uint16)


def test_brute_force_small_special_rows():
    # every row of length <= 4 over a 6-value special alphabet, every k; plus random longer rows
    alpha = np.array([0x0000, 0x8000, 0x7C00, 0xFC00, 0x7E00, 0x3C00], dtype=np.uint16)
    for n in range(1, 5):
        for row in itertools.product(range(len(alpha)), repeat=n):
            bits = alpha[list(row)]
            for k in range(1, n + 2):
                vals, idx = O.batch_topk_half(bits, k, seg_len=n)
                # brute force: rank every element by counting elements that beat it
                keys = O.encode_half_desc_np(bits)
                rank = [sum(1 for j in range(n) if (keys[j], j) < (keys[i], i)) for i in range(n)]
                exp = [rank.index(r) for r in range(min(k, n))]
                assert idx[0, :len(exp)].tolist() == exp
                assert np.all(idx[0, len(exp):] == -1) and np.all(vals[0, len(exp):] == 0xFFFF)
                assert vals[0, :len(exp)].tolist() == bits[exp].tolist()


def test_matches_numpy_lexsort_random():
    rng = np.random.default_rng(7)
    for seg_len, k in [(1, 1), (7, 3), (100, 50), (4096, 50), (5000, 1024)]:
        bits = rng.integers(0, 65536, size=6 * seg_len, dtype=np.uint16)
        bits[rng.random(bits.size) < 0.2] = rng.choice(SPECIALS, size=1)[0]
        v1, i1 = O.batch_topk_half(bits, k, seg_len=seg_len, threads=3)
        v2, i2 = O.topk_lexsort_np(bits, k, seg_len=seg_len)
        np.testing.assert_array_equal(i1, i2)
        np.testing.assert_array_equal(v1, v2)


def test_variable_length_and_padding():
    rng = np.random.default_rng(3)
    lengths = np.array([0, 1, 5, 64, 65, 300], dtype=np.int64)
    offs = np.concatenate([[0], np.cumsum(lengths)])
    bits = rng.integers(0, 65536, size=int(offs[-1]), dtype=np.uint16)
    v1, i1 = O.batch_topk_half(bits, 64, offsets=offs)
    v2, i2 = O.topk_lexsort_np(bits, 64, offsets=offs)
    np.testing.assert_array_equal(i1, i2)
    np.testing.assert_array_equal(v1, v2)
    assert np.all(i1[0] == -1) and np.all(v1[0] == 0xFFFF)
    assert i1[1, 0] == 0 and np.all(i1[1, 1:] == -1)


def test_partial_sort_variant_identical():
    bits = np.random.default_rng(5).integers(0, 65536, size=8 * 3000, dtype=np.uint16)
    t0, i0 = O.time_batch_topk_half(bits, 50, 8, seg_len=3000, variant=0, reps=1)
    t1, i1 = O.time_batch_topk_half(bits, 50, 8, seg_len=3000, variant=1, reps=1, threads=2)
    np.testing.assert_array_equal(i0, i1)
    assert t0 > 0 and t1 > 0


# ------------------------------------------------------------------ radix state helpers

def test_radix_state_kats(kats):
    st = kats["radix_state"]
    s = O.simulate_radix_boundary(st[0]["values"], 8, st[0]["k"])
    for key, val in st[0]["simulate"].items():
        assert s[key] == val, key
    bits = O.float_to_half(np.array(st[0]["values"], dtype=np.float32))
    c = O.cutoff_state(bits, st[0]["k"])
    for key, val in st[0]["cutoff"].items():
        assert c[key] == val, key
    c = O.cutoff_state(bits, st[1]["k"])   # k > len: sentinel (src/radix_boundary_select.cuh:37-45)
    for key, val in st[1]["cutoff"].items():
        assert c[key] == val, key


def test_histogram_kats(kats):
    h = kats["histogram"]
    bits = O.float_to_half(np.array(h["values"], dtype=np.float32))
    hi = O.histogram_pass(bits, 8, 0, 0)
    assert {str(i): int(c) for i, c in enumerate(hi) if c} == h["high_byte"]
    lo = O.histogram_pass(bits, 0, 0x3800, 0xFF00)
    assert {str(i): int(c) for i, c in enumerate(lo) if c} == h["low_byte_in_prefix_0x3800"]


def test_cutoff_brute_force():
    # cutoff key = key of the k-th best element; strictly-better count = #keys < cutoff.
    rng = np.random.default_rng(11)
    for _ in range(200):
        n = int(rng.integers(1, 300))
        k = int(rng.integers(1, n + 1))
        bits = rng.choice(SPECIALS, size=n).astype(np.uint16)
        st = O.cutoff_state(bits, k)
        keys = np.sort(O.encode_half_desc_np(bits).astype(np.int64))
        assert st["cutoff_key"] == keys[k - 1]
        assert st["strictly_better_count"] == int(np.sum(keys < keys[k - 1]))
        assert st["remaining_slots"] == k - st["strictly_better_count"]


# ------------------------------------------------------------------ reference generator

def test_reference_random_generator_rounds_like_numpy():
    v, b = O.make_random_input(2, 1000, 1234)
    assert v.min() >= -64 and v.max() <= 64
    np.testing.assert_array_equal(v.astype(np.float16).view(np.uint16), b)
    v2, b2 = O.make_random_input(2, 1000, 1234)
    np.testing.assert_array_equal(b, b2)
    _, b3 = O.make_random_input(2, 1000, 7)
    assert not np.array_equal(b, b3)


# ------------------------------------------------------------------ bfloat16 extension

BF16_SPECIALS = np.array([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0xFFC1, 0x7F81, 0x3F80, 0xBF80],
                         dtype=np.uint16)


def test_bf16_widening_matches_torch_exhaustive():
    torch = pytest.importorskip("torch")
    bits = np.arange(65536, dtype=np.uint16)
    ours = O.bf16_to_float(bits)
    ref = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours.view(np.uint32), ref.view(np.uint32))


def test_bf16_key_known_answers_and_order():
    # hand-derived: bf16(1.0) = 0x3F80 -> 0x3F80 ^ 0x7FFF; -1.0 keeps its bits; +-inf, NaN, +-0
    assert O.encode_bf16_desc(0x3F80) == 0x407F
    assert O.encode_bf16_desc(0xBF80) == 0xBF80
    assert O.encode_bf16_desc(0x7F80) == 0x007F and O.encode_bf16_desc(0xFF80) == 0xFF80
    for nan in (0x7F81, 0x7FC0, 0xFFC1, 0xFFFF):
        assert O.encode_bf16_desc(nan) == 0xFFFF
    assert O.encode_bf16_desc(0x0000) == O.encode_bf16_desc(0x8000) == 0x7FFF
    bits = np.arange(65536, dtype=np.uint16)
    keys = np.array([O.encode_bf16_desc(int(b)) for b in bits], dtype=np.int64)
    np.testing.assert_array_equal(keys, O.encode_bf16_desc_np(bits).astype(np.int64))
    f = (bits.astype(np.uint32) << 16).view(np.float32)
    nan = np.isnan(f)
    assert np.all(keys[nan] == 0xFFFF)
    fv, kv = f[~nan].astype(np.float64), keys[~nan]
    order = np.argsort(-fv, kind="stable")
    fs, ks = fv[order], kv[order]
    assert np.all(np.diff(ks) >= 0)
    assert np.all((np.diff(ks) == 0) == (np.diff(fs) == 0))


def test_bf16_verifier_matches_numpy_lexsort():
    rng = np.random.default_rng(11)
    for seg_len, k in [(1, 1), (9, 4), (300, 50), (5000, 256)]:
        bits = rng.integers(0, 65536, size=5 * seg_len, dtype=np.uint16)
        bits[rng.random(bits.size) < 0.2] = rng.choice(BF16_SPECIALS, size=1)[0]
        v1, i1 = O.batch_topk_half(bits, k, seg_len=seg_len, threads=2, fmt="bf16")
        v2, i2 = O.topk_lexsort_np(bits, k, seg_len=seg_len, fmt="bf16")
        np.testing.assert_array_equal(i1, i2)
        np.testing.assert_array_equal(v1, v2)


def test_bf16_brute_force_small_rows():
    alpha = BF16_SPECIALS[:7]
    for n in range(1, 4):
        for row in itertools.product(range(len(alpha)), repeat=n):
            bits = alpha[list(row)]
            f = (bits.astype(np.uint32) << 16).view(np.float32)
            # brute force with the reference comparator on floats: NaN last, larger first, index
            def beats(j, i):
                if np.isnan(f[j]) != np.isnan(f[i]):
                    return np.isnan(f[i])
                if not np.isnan(f[j]) and f[j] != f[i]:
                    return f[j] > f[i]
                return j < i
            rank = [sum(1 for j in range(n) if beats(j, i)) for i in range(n)]
            for k in range(1, n + 1):
                _, idx = O.batch_topk_half(bits, k, seg_len=n, fmt="bf16")
                assert idx[0].tolist() == [rank.index(r) for r in range(k)]


# ------------------------------------------------------------------ fp32 (extension)

F32_SPECIALS = np.array([0x7FC00000, 0xFFC00001, 0x7F800001, 0x7FFFFFFF,   # NaNs, both signs
                         0x00000000, 0x80000000, 0x7F800000, 0xFF800000,   # +0, -0, +inf, -inf
                         0x00000001, 0x80000001, 0x007FFFFF, 0x3F800000,   # subnormals, 1.0
                         0xBF800000, 0x3F800001], dtype=np.uint32)


def _f32_bits(values):
    return np.asarray(values, dtype=np.float32).view(np.uint32)


def test_f32_reference_host_kats():
    # test/test_batch_topk.cu:19-44, exact in fp32, through the batched fp32 verifier
    v, i = O.batch_topk_half(_f32_bits([5, 7, 7, 1]), 2, seg_len=4, fmt="f32")
    assert i[0].tolist() == [1, 2] and v[0].view(np.float32).tolist() == [7, 7]
    v, i = O.batch_topk_half(_f32_bits([np.nan, 3, -1, np.nan]), 3, seg_len=4, fmt="f32")
    assert i[0].tolist() == [1, 2, 0] and v[0][2] == _f32_bits([np.nan])[0]
    v, i = O.batch_topk_half(_f32_bits([2, 1]), 4, offsets=np.array([0, 2]), fmt="f32")
    assert i[0].tolist() == [0, 1, -1, -1] and v[0].tolist()[2:] == [0xFFFFFFFF] * 2


def test_f32_key_orders_like_floats():
    # the 32-bit key against float order: every special class and a random sample of patterns
    rng = np.random.default_rng(3)
    bits = np.concatenate([F32_SPECIALS, rng.integers(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32)])
    keys = O.encode_f32_desc_np(bits).astype(np.int64)
    with np.errstate(invalid="ignore"):
        f = bits.view(np.float32).astype(np.float64)
    nan = np.isnan(f)
    assert np.all(keys[nan] == 0xFFFFFFFF) and np.all(keys[~nan] < 0xFFFFFFFF)
    g = f[~nan]
    kg = keys[~nan]
    order = np.argsort(kg, kind="stable")
    assert np.all(np.diff(g[order]) <= 0)                     # ascending key = descending value
    eq = np.diff(kg[order]) == 0
    assert np.all(np.diff(g[order])[eq] == 0)                  # equal keys only for equal values
    assert np.all(np.diff(g[order])[~eq] < 0)                  # distinct values, distinct keys
    assert O.encode_f32_desc_np(np.array([0x00000000, 0x80000000], dtype=np.uint32)).tolist() == [0x7FFFFFFF] * 2


def test_f32_verifier_matches_numpy_lexsort_with_specials():
    rng = np.random.default_rng(11)
    seg_len = 3001
    bits = rng.standard_normal(40 * seg_len).astype(np.float32).view(np.uint32).copy()
    pos = rng.integers(0, bits.size, size=bits.size // 8)
    bits[pos] = F32_SPECIALS[rng.integers(0, F32_SPECIALS.size, size=pos.size)]
    bits[rng.integers(0, bits.size, size=bits.size // 8)] = _f32_bits([1.5])[0]   # ties
    for k in (1, 7, 50, 300):
        got = O.batch_topk_half(bits, k, seg_len=seg_len, fmt="f32", threads=4)
        exp = O.topk_lexsort_np(bits, k, seg_len=seg_len, fmt="f32")
        assert np.array_equal(got[0], exp[0]) and np.array_equal(got[1], exp[1]), k


def test_f32_verifier_agrees_with_fp16_on_widened_rows():
    # fp16 values widen exactly to fp32 and keep their order: the fp32 verifier must select
    # what the (pinned) fp16 verifier selects, with the widened values
    rng = np.random.default_rng(12)
    h = rng.integers(0, 65536, size=30 * 2000).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    for k in (1, 64, 500):
        v16, i16 = O.batch_topk_half(h, k, seg_len=2000)
        v32, i32 = O.batch_topk_half(f.view(np.uint32), k, seg_len=2000, fmt="f32")
        assert np.array_equal(i16, i32), k
        ok = i16 >= 0
        w = v16.view(np.float16).astype(np.float32).view(np.uint32)
        nan = np.isnan(v16.view(np.float16))
        assert np.array_equal(w[ok & ~nan], v32[ok & ~nan]), k   # NaN payloads widen differently


def test_f32_brute_force_small_rows():
    alpha = F32_SPECIALS[[0, 1, 4, 5, 6, 7, 8, 11]]
    for n in range(1, 4):
        for row in itertools.product(range(len(alpha)), repeat=n):
            bits = alpha[list(row)]
            f = bits.view(np.float32)
            def beats(j, i):
                if np.isnan(f[j]) != np.isnan(f[i]):
                    return np.isnan(f[i])
                if not np.isnan(f[j]) and f[j] != f[i]:
                    return f[j] > f[i]
                return j < i
            rank = [sum(1 for j in range(n) if beats(j, i)) for i in range(n)]
            for k in range(1, n + 1):
                v, idx = O.batch_topk_half(bits, k, seg_len=n, fmt="f32")
                assert idx[0].tolist() == [rank.index(r) for r in range(k)]
                assert v[0].tolist() == [int(bits[rank.index(r)]) for r in range(k)]


# ------------------------------------------------------------------ sampling consumer

def test_sample_rule_matches_scipy_softmax():
    special = pytest.importorskip("scipy.special")
    rng = np.random.default_rng(4)
    k = 50
    logits = np.sort(rng.standard_normal((8, k)) * 3, axis=1)[:, ::-1].astype(np.float16)
    bits = logits.view(np.uint16)
    idx = np.tile(np.arange(k, dtype=np.int32), (8, 1))
    for temp in (0.25, 1.0, 3.0):
        _, probs, _, _ = O.sample_topk_np(bits, idx, temp, np.full(8, 0.5))
        inv_t = float(np.float32(1.0) / np.float32(temp))
        ref = special.softmax(logits.astype(np.float64) * inv_t, axis=1)
        np.testing.assert_allclose(probs, ref, rtol=1e-12, atol=1e-15)


def test_sample_rule_closed_forms():
    # k = 1: the only candidate, whatever u
    s, p, _, _ = O.sample_topk_np(np.array([[0x3C00]], np.uint16), np.array([[7]]), 1.0, np.array([0.999]))
    assert s[0] == 7 and p[0, 0] == 1.0
    # equal logits: uniform; u in the j-th 1/m slice picks rank j
    m = 8
    bits = np.full((1, m), 0x4000, np.uint16)
    idx = np.arange(m, dtype=np.int32)[None, :] + 100
    for j in range(m):
        s, p, _, _ = O.sample_topk_np(bits, idx, 0.7, np.array([(j + 0.5) / m]))
        assert s[0] == 100 + j
        np.testing.assert_allclose(p[0], 1.0 / m)
    # two values d apart: p0 = 1 / (1 + exp(-d / T))
    bits = np.array([[np.float16(2.0).view(np.uint16), np.float16(0.5).view(np.uint16)]])
    _, p, _, _ = O.sample_topk_np(bits, np.array([[0, 1]]), 0.5, np.array([0.1]))
    assert abs(p[0, 0] - 1.0 / (1.0 + np.exp(-1.5 / 0.5))) < 1e-12
    # NaN logits get weight 0, -inf gets 0 below a finite best, pads are skipped
    nan, ninf = 0x7E00, 0xFC00
    bits = np.array([[0x3C00, ninf, nan, 0xFFFF]], np.uint16)
    _, p, _, _ = O.sample_topk_np(bits, np.array([[3, 4, 5, -1]]), 1.0, np.array([0.99]))
    assert p[0].tolist() == [1.0, 0.0, 0.0, 0.0]


def test_sample_rule_histogram_on_a_uniform_grid():
    rng = np.random.default_rng(9)
    k, n = 20, 4000
    logits = np.sort(rng.standard_normal(k), kind="stable")[::-1].astype(np.float16)
    bits = np.tile(logits.view(np.uint16), (n, 1))
    idx = np.tile(np.arange(k, dtype=np.int32), (n, 1))
    u = (np.arange(n) + 0.5) / n
    s, p, _, _ = O.sample_topk_np(bits, idx, 1.3, u)
    counts = np.bincount(s, minlength=k)
    assert np.all(np.abs(counts - n * p[0]) <= 1.0 + 1e-9)
