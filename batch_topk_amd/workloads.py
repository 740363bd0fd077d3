"""Deterministic synthetic fp16 workloads (numpy PCG64, seed 0 unless stated).

The five workloads the engine is measured and checked on:

* ``uniform_small``    16 x 4096, U(-1, 1), k = 50.
* ``llm_logits``       128 x 128256, N(0, sd 2) with 0.1 % of each row (128 positions)
                       boosted by +8 before fp16 rounding, k = 50.
* ``varlen``           512 segments, lengths U{1..65536} with segments 0-7 forced to
                       {1, 2, 31, 49, 50, 63, 64, 65}, N(0, 1), int32 offsets, k = 64.
* ``ties_special``     256 x 32000 drawn from 256 distinct values (j - 128) / 32 with a random
                       sign on every zero, 1 % -inf and 0.1 % NaN per row (bit patterns
                       0x7E00, 0xFE00, 0x7C01, 0xFFFF in turn), k in {1, 16, 128, 256}.
* ``huge_segment``     1 x 16,777,216, N(0, 1), k = 1024.

And the reference's own benchmark matrix (``ref_matrix``): seg_num in {128, 1500, 3000, 4500,
6000} x 10000, k = 50, filled as the reference's bench fills its input
(bench/bench_batch_topk.cu:9-15: element i = ((i * 17 + 13) mod 2048 - 1024) / 16 over the
whole batch, exact in fp16), with the reference's RTX 4080 targets
(include/batch_topk_benchmark.cuh:14-20).

Every generator returns raw fp16 bit patterns (uint16) so that NaN payloads and the sign of
zero survive; float -> fp16 conversion is numpy's round-to-nearest-even cast.
"""

from __future__ import annotations

import numpy as np

NEG_INF = 0xFC00
NAN_PATTERNS = (0x7E00, 0xFE00, 0x7C01, 0xFFFF)


def _f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def uniform_small(seed: int = 0, seg_num: int = 16, seg_len: int = 4096):
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1.0, 1.0, size=(seg_num, seg_len)).astype(np.float32)
    return _f16_bits(x)


def llm_logits(seed: int = 0, seg_num: int = 128, seg_len: int = 128256, boost_frac: float = 0.001,
               boost: float = 8.0, sd: float = 2.0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((seg_num, seg_len), dtype=np.float32) * np.float32(sd)
    n_boost = int(round(boost_frac * seg_len))
    for s in range(seg_num):
        pos = rng.choice(seg_len, size=n_boost, replace=False)
        x[s, pos] += np.float32(boost)
    return _f16_bits(x)


def varlen(seed: int = 0, seg_num: int = 512, max_len: int = 65536,
           forced=(1, 2, 31, 49, 50, 63, 64, 65)):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(1, max_len + 1, size=seg_num).astype(np.int64)
    lengths[: len(forced)] = forced[: seg_num]
    offsets = np.zeros(seg_num + 1, dtype=np.int64)
    np.cumsum(lengths, out=offsets[1:])
    x = rng.standard_normal(int(offsets[-1]), dtype=np.float32)
    return _f16_bits(x), offsets.astype(np.int32)


def ties_special(seed: int = 0, seg_num: int = 256, seg_len: int = 32000):
    rng = np.random.default_rng(seed)
    table = ((np.arange(256, dtype=np.float32) - 128.0) / 32.0)
    tbits = _f16_bits(table)
    pick = rng.integers(0, 256, size=(seg_num, seg_len))
    bits = tbits[pick]
    zero = pick == 128
    signs = rng.integers(0, 2, size=(seg_num, seg_len)).astype(bool)
    bits = np.where(zero & signs, np.uint16(0x8000), bits).astype(np.uint16)
    n_inf = int(round(0.01 * seg_len))
    n_nan = int(round(0.001 * seg_len))
    for s in range(seg_num):
        pos = rng.choice(seg_len, size=n_inf + n_nan, replace=False)
        bits[s, pos[:n_inf]] = NEG_INF
        nan_pos = pos[n_inf:]
        bits[s, nan_pos] = np.array([NAN_PATTERNS[i % 4] for i in range(n_nan)], dtype=np.uint16)
    return bits


def huge_segment(seed: int = 0, n: int = 16_777_216):
    rng = np.random.default_rng(seed)
    return _f16_bits(rng.standard_normal((1, n), dtype=np.float32))


# (seg_num, seg_len, k) -> target latency in us on RTX 4080 (include/batch_topk_benchmark.cuh:14-20)
REF_MATRIX_TARGET_US = {
    (128, 10000, 50): 11.0,
    (1500, 10000, 50): 82.0,
    (3000, 10000, 50): 161.0,
    (4500, 10000, 50): 241.0,
    (6000, 10000, 50): 319.0,
}


def ref_matrix(seg_num: int = 128, seg_len: int = 10000):
    i = np.arange(seg_num * seg_len, dtype=np.int64)
    raw = (i * 17 + 13) % 2048 - 1024
    return _f16_bits((raw.astype(np.float32) / np.float32(16.0)).reshape(seg_num, seg_len))


WORKLOADS = {
    "uniform_small": dict(gen=uniform_small, k=(50,)),
    "llm_logits": dict(gen=llm_logits, k=(50,)),
    "varlen": dict(gen=varlen, k=(64,)),
    "ties_special": dict(gen=ties_special, k=(1, 16, 128, 256)),
    "huge_segment": dict(gen=huge_segment, k=(1024,)),
    "ref_matrix": dict(gen=ref_matrix, k=(50,)),
}
