"""A C++ caller of the reference's host API, run on the GPU through the drop-in header.

tests/cpp/dropin_caller.cpp includes include/batch_topk.hpp and calls
radix_topk::batch_topk_half / batch_topk_half_workspace_size exactly as a caller of the
reference (include/batch_topk.cuh:10-21) does, spelled with HIP types.  It first replays the
reference's API sequence (test/test_batch_topk.cu:1302-1385: NULL pointers and k > seg_len
rejected with hipErrorInvalidValue, a workspace one byte short rejected, then a successful call
on a zero row), then runs every golden case of tests/golden/kats.json (the poisoned one with a
0xA5-filled workspace) and two seeded workloads, whose answers come from the oracle.  The
binary is built by batch_topk_amd/build.py next to its source and started as a child process."""

import json
import os
import subprocess

import numpy as np
import pytest

import batch_topk_amd as bt
from batch_topk_amd import build as hip_build
from batch_topk_amd import workloads as wl
from oracle import oracle as O
from tests.gpu_util import announce

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "kats.json")


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    bt.load_library()


def test_cpp_caller_through_dropin_header(tmp_path):
    if not os.path.exists(hip_build.CPP_CALLER_BIN):
        pytest.fail(f"{hip_build.CPP_CALLER_BIN} is missing: run python -m batch_topk_amd.build")
    with open(GOLDEN) as f:
        golden = json.load(f)["cases"]
    cases = []  # (name, bits [seg_num, seg_len], k, poison, expected indices, expected value bits)
    for c in golden:
        bits = np.array(c["input_bits"], dtype=np.uint16).reshape(c["seg_num"], c["seg_len"])
        cases.append((c["name"], bits, c["k"], "poisoned" in c["name"],
                      np.array(c["expected_idx"]), np.array(c["expected_val_bits"])))
    rng = np.random.default_rng(3)
    for name, bits, k in (("uniform_small_16x4096", wl.uniform_small(), 50),
                          ("logits_4x130000", wl.llm_logits(seg_num=4, seg_len=130000), 64),
                          ("ties_8x32000_k256", wl.ties_special(seg_num=8), 256),
                          ("normal_2x300000_k700",
                           rng.standard_normal((2, 300000)).astype(np.float16).view(np.uint16), 700)):
        ev, ei = O.batch_topk_half(bits, k, seg_len=bits.shape[1], threads=8)
        cases.append((name, bits, k, True, ei, ev))
    path = tmp_path / "cases.txt"
    with open(path, "w") as f:
        f.write(f"{len(cases)}\n")
        for name, bits, k, poison, _, _ in cases:
            f.write(f"{name} {bits.shape[0]} {bits.shape[1]} {k} {int(poison)}\n")
            f.write(" ".join(map(str, bits.reshape(-1).tolist())) + "\n")
    announce(f"C++ drop-in caller: API sequence and {len(cases)} cases")
    res = subprocess.run([hip_build.CPP_CALLER_BIN, str(path)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    lines = res.stdout.splitlines()
    assert lines[0] == "api ok", lines[:3]
    for i, (name, bits, k, _, ei, ev) in enumerate(cases):
        head, idx_line, val_line = lines[1 + 3 * i: 4 + 3 * i]
        assert head == f"case {name}"
        gi = np.array(idx_line.split(), dtype=np.int64).reshape(bits.shape[0], k)
        gv = np.array(val_line.split(), dtype=np.int64).reshape(bits.shape[0], k)
        assert np.array_equal(gi, np.asarray(ei).reshape(bits.shape[0], k)), name
        assert np.array_equal(gv, np.asarray(ev).reshape(bits.shape[0], k)), name
