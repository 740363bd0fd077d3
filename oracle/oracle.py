"""Parity oracle for the batched fp16 / bf16 top-k path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import this module, and only as the checker or as the timed CPU baseline.  The
product path (``batch_topk_amd``) never imports it.

Two independent restatements live here:

* ``liboracle.so`` (built from ``oracle.cpp``): the reference's host verifier
  ``cpu_reference_topk`` (include/batch_topk_types.cuh:50-92, a ``std::stable_sort`` with
  the NaN-last comparator), the codec (include/type_codec.cuh:9-38), the comparator
  (include/batch_topk_types.cuh:100-113) and the radix-state helpers
  (src/radix_select_state.cuh:9-51, src/radix_boundary_select.cuh:9-78).
* numpy functions below (``encode_half_desc_np``, ``topk_lexsort_np``): a second,
  differently-built statement of the same order (sort by the order-preserving 16-bit
  key, then by index) used to cross-check the C++ restatement on large random inputs.

How each oracle function is pinned (tests/test_oracle.py):

* codec: the known answers derived from the reference tests (desc(3.0)=0x3DFF,
  desc(-1.0)=0xBC00, desc(+-0)=0x7FFF, desc(+inf)=0x03FF, desc(-inf)=0xFC00,
  desc(NaN)=0xFFFF, test/test_batch_topk.cu:46-51) and, over all 65536 bit patterns,
  monotonicity against numpy's float16 ordering (closed form of IEEE-754 binary16).
* cpu_reference_topk: the reference's host KATs (test/test_batch_topk.cu:19-44), the
  hand-derived end-to-end answers of test/test_batch_topk.cu:332-425, 602-710, 712-815
  and 922-1026 (committed under tests/golden/), brute force over all small inputs drawn
  from special values, and the numpy lexsort restatement on random data.
* simulate_radix_boundary / select / finalize: the reference's state KATs
  (test/test_batch_topk.cu:66-74, 169-201, 203-234) and a brute-force cumulative count.
* half <-> float conversions: numpy's float16 casts over every bit pattern.
* fp32 (an extension): the verifier itself compares floats, so the batched fp32 oracle is
  the reference's verifier on the input floats; it is checked against the numpy lexsort
  restatement with the 32-bit key (``encode_f32_desc_np``) on random data with NaN payloads,
  +-0, +-inf and subnormals, the key against float order on every special class and a
  large random sample, and the reference's own host KATs (exact in fp32).
* bfloat16 (an extension: the reference covers fp16 only): the bf16 -> float widening
  against torch's bfloat16 cast over every bit pattern; the bf16 key against float order
  over every bit pattern and hand-derived known answers; the batched bf16 verifier against
  the numpy lexsort restatement with the bf16 key on random data with special values.
* sample_topk_np (the sampling consumer, an extension with no reference counterpart): the
  softmax weights against scipy.special.softmax, closed forms (k = 1, equal logits, the
  two-value logistic), and a deterministic grid of uniforms whose sampled-rank histogram
  must equal the probabilities times the grid size.  It is floating point: GPU results are
  compared to it with the tolerances stated in tests/test_sample_gpu.py.
* make_random_input: bit patterns are checked against numpy's RNE float16 cast of the
  same floats; the stream itself is libstdc++'s mt19937, as in the reference's tests.

Nothing in this module is "parity unpinned" except the pad convention for ranks beyond
a short segment's length (index -1, value 0xFFFF), which the reference does not define
(it rejects k > seg_len).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

PAD_INDEX = -1
PAD_VALUE_BITS = 0xFFFF


def build(force: bool = False) -> str:
    """Compile oracle.cpp into liboracle.so with the committed Makefile."""
    cmd = ["make", "-s"] + (["-B"] if force else []) + ["liboracle.so"]
    subprocess.run(cmd, cwd=_HERE, check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        u16, i32, i64, f32, f64 = (ctypes.c_uint16, ctypes.c_int32, ctypes.c_int64,
                                   ctypes.c_float, ctypes.c_double)
        vp = ctypes.c_void_p
        L.oracle_normalize_half_bits.restype = u16
        L.oracle_normalize_half_bits.argtypes = [u16]
        L.oracle_encode_half_asc.restype = u16
        L.oracle_encode_half_asc.argtypes = [u16]
        L.oracle_encode_half_desc.restype = u16
        L.oracle_encode_half_desc.argtypes = [u16]
        L.oracle_half_to_float.restype = f32
        L.oracle_half_to_float.argtypes = [u16]
        L.oracle_float_to_half.restype = u16
        L.oracle_float_to_half.argtypes = [f32]
        L.oracle_half_to_float_array.restype = None
        L.oracle_half_to_float_array.argtypes = [vp, i64, vp]
        L.oracle_float_to_half_array.restype = None
        L.oracle_float_to_half_array.argtypes = [vp, i64, vp]
        L.oracle_candidate_better.restype = ctypes.c_int
        L.oracle_candidate_better.argtypes = [u16, ctypes.c_int, u16, ctypes.c_int]
        L.oracle_cpu_reference_topk.restype = ctypes.c_int
        L.oracle_cpu_reference_topk.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
        L.oracle_simulate_radix_boundary.restype = None
        L.oracle_simulate_radix_boundary.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
        L.oracle_select_high_byte_boundary.restype = None
        L.oracle_select_high_byte_boundary.argtypes = [vp, ctypes.c_int, vp]
        L.oracle_finalize_cutoff_key.restype = None
        L.oracle_finalize_cutoff_key.argtypes = [vp, ctypes.c_int, vp]
        L.oracle_histogram_pass.restype = None
        L.oracle_histogram_pass.argtypes = [vp, ctypes.c_int, ctypes.c_int, u16, u16, vp]
        L.oracle_encode_bf16_desc.restype = u16
        L.oracle_encode_bf16_desc.argtypes = [u16]
        L.oracle_bf16_to_float_array.restype = None
        L.oracle_bf16_to_float_array.argtypes = [vp, i64, vp]
        L.oracle_batch_topk_bf16.restype = ctypes.c_int
        L.oracle_batch_topk_bf16.argtypes = [vp, vp, ctypes.c_int, i64, ctypes.c_int, vp, vp,
                                             ctypes.c_int]
        L.oracle_batch_topk_f32.restype = ctypes.c_int
        L.oracle_batch_topk_f32.argtypes = [vp, vp, ctypes.c_int, i64, ctypes.c_int, vp, vp,
                                            ctypes.c_int]
        L.oracle_batch_topk_half.restype = ctypes.c_int
        L.oracle_batch_topk_half.argtypes = [vp, vp, ctypes.c_int, i64, ctypes.c_int, vp, vp,
                                             ctypes.c_int]
        L.oracle_time_batch_topk_half.restype = f64
        L.oracle_time_batch_topk_half.argtypes = [vp, vp, ctypes.c_int, i64, ctypes.c_int,
                                                  ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
        L.oracle_make_random_input.restype = None
        L.oracle_make_random_input.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_uint32, vp, vp]
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


# ---------------------------------------------------------------- C restatement wrappers

def encode_half_desc(bits: int) -> int:
    return int(lib().oracle_encode_half_desc(bits & 0xFFFF))


def encode_half_asc(bits: int) -> int:
    return int(lib().oracle_encode_half_asc(bits & 0xFFFF))


def normalize_half_bits(bits: int) -> int:
    return int(lib().oracle_normalize_half_bits(bits & 0xFFFF))


def encode_bf16_desc(bits: int) -> int:
    return int(lib().oracle_encode_bf16_desc(bits & 0xFFFF))


def bf16_to_float(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    lib().oracle_bf16_to_float_array(_ptr(bits), bits.size, _ptr(out))
    return out


def candidate_better(lhs_bits: int, lhs_index: int, rhs_bits: int, rhs_index: int) -> bool:
    return bool(lib().oracle_candidate_better(lhs_bits, lhs_index, rhs_bits, rhs_index))


def half_to_float(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    lib().oracle_half_to_float_array(_ptr(bits), bits.size, _ptr(out))
    return out


def float_to_half(values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(values.shape, dtype=np.uint16)
    lib().oracle_float_to_half_array(_ptr(values), values.size, _ptr(out))
    return out


def cpu_reference_topk(values, seg_len: int, k: int):
    """include/batch_topk_types.cuh:50-92 on a float vector -> (values list, indices list)."""
    v = np.ascontiguousarray(values, dtype=np.float32)
    n_out = max(0, min(k, seg_len, v.size))
    ov = np.zeros(max(n_out, 1), dtype=np.float32)
    oi = np.zeros(max(n_out, 1), dtype=np.int32)
    got = lib().oracle_cpu_reference_topk(_ptr(v), int(v.size), int(seg_len), int(k), _ptr(ov), _ptr(oi))
    return ov[:got].tolist(), oi[:got].tolist()


STATE_FIELDS = ("prefix", "prefix_mask", "cutoff_key", "selected_count", "live_count",
                "boundary_digit", "strictly_better_count", "remaining_slots")


def simulate_radix_boundary(values, seg_len: int, k: int) -> dict:
    v = np.ascontiguousarray(values, dtype=np.float32)
    st = np.zeros(8, dtype=np.int32)
    lib().oracle_simulate_radix_boundary(_ptr(v), int(v.size), int(seg_len), int(k), _ptr(st))
    return dict(zip(STATE_FIELDS, st.tolist()))


def histogram_pass(bits: np.ndarray, shift: int, prefix: int, mask: int) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    h = np.zeros(256, dtype=np.uint32)
    lib().oracle_histogram_pass(_ptr(bits), int(bits.size), int(shift), prefix, mask, _ptr(h))
    return h


def cutoff_state(bits: np.ndarray, k: int) -> dict:
    """K1 -> K6 -> K2 -> K7 of the reference (high-byte select, then cutoff finalisation)."""
    hist_hi = histogram_pass(bits, 8, 0, 0)
    st = np.zeros(8, dtype=np.int32)
    lib().oracle_select_high_byte_boundary(_ptr(hist_hi), int(k), _ptr(st))
    digit = int(st[5])
    keys = encode_half_desc_np(np.asarray(bits, dtype=np.uint16))
    hist_lo = np.zeros(256, dtype=np.uint32)
    sel = (keys >> 8) == digit
    np.add.at(hist_lo, (keys[sel] & 0xFF).astype(np.int64), 1)
    lib().oracle_finalize_cutoff_key(_ptr(hist_lo), int(k), _ptr(st))
    return dict(zip(STATE_FIELDS, st.tolist()))


def batch_topk_half(bits: np.ndarray, k: int, seg_len: int | None = None,
                    offsets: np.ndarray | None = None, threads: int = 1, fmt: str = "f16"):
    """Reference order on every segment -> (values uint16 [S,k], indices int32 [S,k]).

    Values are the raw input bits at the selected index; ranks beyond a segment's length
    are padded with (PAD_VALUE_BITS, PAD_INDEX).  ``fmt`` is "f16" (the reference's format),
    "bf16" (the same verifier on bfloat16 bits) or "f32" (the verifier on the floats
    themselves: uint32 bits in, uint32 values out, pads 0xFFFFFFFF).
    """
    wide = fmt == "f32"
    bits = np.ascontiguousarray(bits, dtype=np.uint32 if wide else np.uint16).reshape(-1)
    if offsets is not None:
        off = np.ascontiguousarray(offsets, dtype=np.int64)
        seg_num = off.size - 1
        sl = 0
    else:
        assert seg_len is not None and seg_len > 0
        off = None
        seg_num = bits.size // seg_len
        sl = seg_len
    vals = np.empty((seg_num, k), dtype=np.uint32 if wide else np.uint16)
    idx = np.empty((seg_num, k), dtype=np.int32)
    fn = {"f16": lib().oracle_batch_topk_half, "bf16": lib().oracle_batch_topk_bf16,
          "f32": lib().oracle_batch_topk_f32}[fmt]
    rc = fn(_ptr(bits), _ptr(off) if off is not None else None, int(seg_num), int(sl), int(k),
            _ptr(vals), _ptr(idx), int(threads))
    if rc != 0:
        raise ValueError("oracle rejected the arguments")
    return vals, idx


def time_batch_topk_half(bits: np.ndarray, k: int, seg_count: int, seg_len: int | None = None,
                         offsets: np.ndarray | None = None, threads: int = 1, variant: int = 0,
                         reps: int = 3):
    """Median wall seconds of the verifier over the first ``seg_count`` segments."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
    off = np.ascontiguousarray(offsets, dtype=np.int64) if offsets is not None else None
    idx = np.empty((seg_count, k), dtype=np.int32)
    t = lib().oracle_time_batch_topk_half(_ptr(bits), _ptr(off) if off is not None else None,
                                          int(seg_count), int(seg_len or 0), int(k), int(threads),
                                          int(variant), int(reps), _ptr(idx))
    return float(t), idx


def make_random_input(seg_num: int, seg_len: int, seed: int):
    """test/test_batch_topk.cu:446-454 -> (float32 values, uint16 bits)."""
    n = seg_num * seg_len
    v = np.empty(n, dtype=np.float32)
    b = np.empty(n, dtype=np.uint16)
    lib().oracle_make_random_input(int(seg_num), int(seg_len), int(seed) & 0xFFFFFFFF, _ptr(v), _ptr(b))
    return v, b


# ---------------------------------------------------------------- numpy restatement

def encode_half_desc_np(bits: np.ndarray) -> np.ndarray:
    """Order-preserving descending key (include/type_codec.cuh:9-38), vectorised."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32)
    mag = b & 0x7FFF
    nan = mag > 0x7C00
    zero = mag == 0
    neg = (b & 0x8000) != 0
    key = np.where(neg, b, b ^ 0x7FFF)
    key = np.where(zero, 0x7FFF, key)
    key = np.where(nan, 0xFFFF, key)
    return key.astype(np.uint16)


def encode_bf16_desc_np(bits: np.ndarray) -> np.ndarray:
    """The same key for bfloat16 bits (inf = 0x7F80; a larger magnitude is a NaN)."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32)
    mag = b & 0x7FFF
    key = np.where((b & 0x8000) != 0, b, b ^ 0x7FFF)
    key = np.where(mag == 0, 0x7FFF, key)
    key = np.where(mag > 0x7F80, 0xFFFF, key)
    return key.astype(np.uint16)


def encode_f32_desc_np(bits: np.ndarray) -> np.ndarray:
    """The same key for fp32 bits: NaN -> 0xFFFFFFFF, +-0 -> 0x7FFFFFFF, negative -> bits,
    positive -> bits ^ 0x7FFFFFFF."""
    b = np.asarray(bits, dtype=np.uint32).astype(np.uint64)
    mag = b & 0x7FFFFFFF
    key = np.where((b & 0x80000000) != 0, b, b ^ 0x7FFFFFFF)
    key = np.where(mag == 0, 0x7FFFFFFF, key)
    key = np.where(mag > 0x7F800000, 0xFFFFFFFF, key)
    return key.astype(np.uint32)


def topk_lexsort_np(bits: np.ndarray, k: int, seg_len: int | None = None,
                    offsets: np.ndarray | None = None, fmt: str = "f16"):
    """Independent numpy statement of the order: ascending (desc key, index)."""
    encode = {"f16": encode_half_desc_np, "bf16": encode_bf16_desc_np, "f32": encode_f32_desc_np}[fmt]
    wide = fmt == "f32"
    bits = np.asarray(bits, dtype=np.uint32 if wide else np.uint16).reshape(-1)
    if offsets is None:
        seg_num = bits.size // seg_len
        offsets = np.arange(seg_num + 1, dtype=np.int64) * seg_len
    offsets = np.asarray(offsets, dtype=np.int64)
    seg_num = offsets.size - 1
    vals = np.full((seg_num, k), 0xFFFFFFFF if wide else PAD_VALUE_BITS,
                   dtype=np.uint32 if wide else np.uint16)
    idx = np.full((seg_num, k), PAD_INDEX, dtype=np.int32)
    for s in range(seg_num):
        seg = bits[offsets[s]:offsets[s + 1]]
        n = seg.size
        if n == 0:
            continue
        keys = encode(seg)
        order = np.lexsort((np.arange(n), keys))[:k]
        m = order.size
        idx[s, :m] = order
        vals[s, :m] = seg[order]
    return vals, idx


# ---------------------------------------------------------------- sampling consumer

def bits_to_float64(bits: np.ndarray, fmt: str = "f16") -> np.ndarray:
    """Exact widening of fp16 / bfloat16 bit patterns to float64."""
    b = np.asarray(bits, dtype=np.uint16)
    if fmt == "f16":
        return b.view(np.float16).astype(np.float64)
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def sample_topk_np(vals_bits: np.ndarray, idx: np.ndarray, temperature: float,
                   uniforms: np.ndarray, fmt: str = "f16"):
    """The sampling rule of include/batch_topk.h (radix_topk_sample_*), in float64, on a top-k
    output [S, k] (values in rank order, indices with -1 past a short segment).

    -> (samples int32 [S], probs float64 [S, k], cumulative sums float64 [S, k], totals [S]).
    1 / temperature is rounded to float32 first, as the library does on the host.
    """
    v = bits_to_float64(vals_bits, fmt)
    idx = np.asarray(idx)
    inv_t = float(np.float32(1.0) / np.float32(temperature))
    S, k = v.shape
    samples = np.full(S, -1, dtype=np.int32)
    probs = np.zeros((S, k))
    cums = np.zeros((S, k))
    totals = np.zeros(S)
    for s in range(S):
        m = int(np.sum(idx[s] >= 0))
        if m == 0:
            continue
        w = np.zeros(k)
        w[0] = 1.0
        with np.errstate(invalid="ignore", over="ignore"):
            for r in range(1, m):
                if v[s, r] == v[s, 0]:
                    w[r] = 1.0
                else:
                    x = np.exp((v[s, r] - v[s, 0]) * inv_t)
                    w[r] = 0.0 if np.isnan(x) else x
        c = np.cumsum(w)
        total = c[m - 1]
        target = float(uniforms[s]) * total
        hits = np.nonzero(c[:m] > target)[0]
        r = int(hits[0]) if hits.size else m - 1
        samples[s] = idx[s, r]
        probs[s] = w / total
        cums[s] = c
        totals[s] = total
    return samples, probs, cums, totals
