"""Writes tests/golden/kats.json: known-answer vectors taken from the reference's tests.

Every expected answer here is derived from the closed form of the reference test's input
(the reasoning is in the comments), not computed by the oracle, so that the oracle and the
GPU path are both checked against an independent statement.  Inputs are stored as fp16 bit
patterns (numpy's round-to-nearest-even cast, which is what __float2half does for these
exactly-representable values).

Run:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
INF = 0x7C00
NINF = 0xFC00
QNAN = 0x7E00


def f16(vals):
    return [int(b) for b in np.asarray(vals, dtype=np.float32).astype(np.float16).view(np.uint16)]


def case(name, source, seg_num, seg_len, k, bits, exp_idx, note=""):
    bits = [int(b) for b in bits]
    exp_val = []
    for s in range(seg_num):
        row = [bits[s * seg_len + i] for i in exp_idx[s]]
        exp_val.append(row)
    return dict(name=name, source=source, seg_num=seg_num, seg_len=seg_len, k=k,
                input_bits=bits, expected_idx=exp_idx, expected_val_bits=exp_val, note=note)


def main():
    cases = []

    # test/test_batch_topk.cu:19-25 -- {5,7,7,1}, k=2: the two 7s, lower index first.
    cases.append(case("reference_ordering", "test/test_batch_topk.cu:19-25", 1, 4, 2,
                      f16([5, 7, 7, 1]), [[1, 2]]))

    # test/test_batch_topk.cu:27-36 -- {NaN,3,-1,NaN}, k=3: 3, -1, then the first NaN.
    cases.append(case("reference_nan_ordering", "test/test_batch_topk.cu:27-36", 1, 4, 3,
                      [QNAN] + f16([3, -1]) + [QNAN], [[1, 2, 0]]))

    # test/test_batch_topk.cu:332-425 -- 2 x 8, k = 3.
    seg0 = [1, 9, 2, 8, 3, 7, 4, 6]   # 9@1, 8@3, 7@5
    seg1 = [5, 4, 9, 1, 9, 2, 0, 8]   # 9@2, 9@4 (tie -> index order), 8@7
    cases.append(case("gpu_small_correctness", "test/test_batch_topk.cu:332-425", 2, 8, 3,
                      f16(seg0 + seg1), [[1, 3, 5], [2, 4, 7]]))

    # test/test_batch_topk.cu:602-710 -- 64 values: 42,42,+inf,+inf,17,17,NaN,-inf, then -i.
    # Order: +inf@2,+inf@3, 42@0,42@1, 17@4,17@5, then -8@8 ... -51@51 (44 entries) = 50.
    vals = [float(-i) for i in range(64)]
    bits = f16(vals)
    bits[0:8] = f16([42, 42])[0:2] + [INF, INF] + f16([17, 17]) + [QNAN, NINF]
    cases.append(case("final_topk50_ordering", "test/test_batch_topk.cu:602-710", 1, 64, 50,
                      bits, [[2, 3, 0, 1, 4, 5] + list(range(8, 52))]))

    # test/test_batch_topk.cu:477-496,712-815 -- 2 x 10000, k = 50.  Base value
    # -512 + (i+s) % 113 in [-512, -400]; +inf at 3 and 9, 2048-s at 15 and 21, 1024+s at 27,
    # -inf at 33, NaN at 39 and 45.  Order: 3, 9, 15, 21, 27, then the largest base value -400,
    # reached where (i + s) % 113 == 112, in index order (45 of them).
    seg_num, seg_len = 2, 10000
    allb, exp = [], []
    for s in range(seg_num):
        row = [-512.0 + float((i + s) % 113) for i in range(seg_len)]
        rb = f16(row)
        rb[3] = INF
        rb[9] = INF
        rb[15] = f16([2048 - s])[0]
        rb[21] = f16([2048 - s])[0]
        rb[27] = f16([1024 + s])[0]
        rb[33] = NINF
        rb[39] = QNAN
        rb[45] = QNAN
        allb += rb
        tail = [i for i in range(seg_len) if (i + s) % 113 == 112][:45]
        exp.append([3, 9, 15, 21, 27] + tail)
    cases.append(case("optimized_nan_inf", "test/test_batch_topk.cu:477-496,712-815",
                      seg_num, seg_len, 50, allb, exp))

    # test/test_batch_topk.cu:456-471,922-1026 -- 4 x 10000, k = 50, workspace poisoned 0xa5.
    # i < 64: 200 - (64 s + i); else ((i + s) % 5) - 2 in [-2, 2].
    # s = 0,1,2: the 64 leading values are all > 2 and decreasing -> indices 0..49.
    # s = 3: leading values 8 - i; 8..3 at i = 0..5 beat every tail value, 2 at i = 6 ties the
    # tail maximum 2 (reached at i % 5 == 1, i >= 64) and wins on index; then 66, 71, ...
    seg_num, seg_len = 4, 10000
    allb, exp = [], []
    for s in range(seg_num):
        row = [200.0 - (s * 64 + i) if i < 64 else float(((i + s) % 5) - 2) for i in range(seg_len)]
        allb += f16(row)
        if s < 3:
            exp.append(list(range(50)))
        else:
            exp.append(list(range(7)) + [66 + 5 * j for j in range(43)])
    cases.append(case("duplicate_heavy_poisoned", "test/test_batch_topk.cu:456-471,922-1026",
                      seg_num, seg_len, 50, allb, exp, note="workspace filled with 0xa5 before the call"))

    out = dict(
        generated_by="tests/golden/make_golden.py",
        cases=cases,
        codec_desc=[  # test/test_batch_topk.cu:46-51 and the closed form of type_codec.cuh
            [f16([3.0])[0], 0x3DFF], [f16([-1.0])[0], 0xBC00], [f16([9.0])[0], 0x377F],
            [f16([7.0])[0], 0x38FF], [0x0000, 0x7FFF], [0x8000, 0x7FFF], [INF, 0x03FF],
            [NINF, 0xFC00], [QNAN, 0xFFFF], [0xFE00, 0xFFFF], [0x7C01, 0xFFFF], [0xFFFF, 0xFFFF],
        ],
        radix_state=[  # test/test_batch_topk.cu:66-74, 169-201 on {9,8,...,2}
            dict(values=[9, 8, 7, 6, 5, 4, 3, 2], k=3,
                 simulate=dict(selected_count=2, live_count=1, boundary_digit=56, prefix=0x3800,
                               prefix_mask=0xFF00),
                 cutoff=dict(strictly_better_count=2, remaining_slots=1, cutoff_key=0x38FF)),
            dict(values=[9, 8, 7, 6, 5, 4, 3, 2], k=9,
                 cutoff=dict(prefix=0xFFFF, prefix_mask=0xFFFF, cutoff_key=0xFFFF, live_count=0,
                             boundary_digit=255, strictly_better_count=8, remaining_slots=1)),
        ],
        histogram=dict(  # test/test_batch_topk.cu:203-234
            values=[9, 8, 7, 6, 5, 4, 3, 2],
            high_byte={"55": 2, "56": 1, "57": 1, "58": 1, "59": 1, "61": 1, "63": 1},
            low_byte_in_prefix_0x3800={"255": 1}),
    )
    path = os.path.join(HERE, "kats.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
