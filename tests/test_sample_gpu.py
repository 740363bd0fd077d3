"""GPU checks of the top-k sampling consumer (radix_topk_sample_half / _bf16) through the C ABI.

The top-k part is integer work and must be bit-exact with the oracle.  The sampling part is
fp32 floating point (exp, a sum over up to 1024 weights), so it is compared with the oracle's
float64 statement of the same rule (oracle.sample_topk_np) within stated tolerances:
  * probabilities: |gpu - ref| <= PROB_RTOL * ref + PROB_ATOL;
  * sampled index: the pick's rank r must satisfy cum[r-1] - TOL <= u * S <= cum[r] + TOL with
    TOL = SAMPLE_RTOL * S (cum, S from the oracle), and must equal the oracle's pick whenever
    u * S is farther than TOL from every cumulative boundary.
"""

import numpy as np
import pytest

import batch_topk_amd as bt
from batch_topk_amd import workloads as wl
from oracle import oracle as O
from tests.gpu_util import announce, device_u16

pytestmark = pytest.mark.gpu

PROB_RTOL, PROB_ATOL = 1e-4, 1e-7
SAMPLE_RTOL = 1e-4
THREADS = 8


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    bt.load_library()


def run_sample(bits, k, temperature, u, fmt="f16", with_probs=True):
    import torch

    seg_num, seg_len = bits.shape
    fn, wsf = (bt.sample_half, bt.sample_half_workspace_size) if fmt == "f16" else \
        (bt.sample_bf16, bt.sample_bf16_workspace_size)
    buf = device_u16(bits)
    ws_bytes = wsf(seg_num, seg_len, k)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
    vals = torch.empty((seg_num, k), dtype=torch.int16, device="cuda:0")
    idx = torch.empty((seg_num, k), dtype=torch.int32, device="cuda:0")
    probs = torch.full((seg_num, k), -1.0, dtype=torch.float32, device="cuda:0")
    samples = torch.full((seg_num,), -7, dtype=torch.int32, device="cuda:0")
    du = torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).to("cuda:0")
    rc = fn(buf.data_ptr(), seg_num, seg_len, k, temperature, du.data_ptr(), vals.data_ptr(),
            idx.data_ptr(), probs.data_ptr() if with_probs else 0, samples.data_ptr(), ws.data_ptr(),
            ws_bytes, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return (vals.cpu().numpy().view(np.uint16), idx.cpu().numpy(), probs.cpu().numpy(),
            samples.cpu().numpy())


def check_sample(bits, k, temperature, u, what, fmt="f16"):
    announce(f"sample {what} {fmt} shape={bits.shape} k={k} T={temperature}")
    vals, idx, probs, samples = run_sample(bits, k, temperature, u, fmt)
    ev, ei = O.batch_topk_half(bits, k, seg_len=bits.shape[1], threads=THREADS, fmt=fmt)
    assert np.array_equal(idx, ei) and np.array_equal(vals, ev), f"{what}: top-k not bit-exact"
    es, ep, cum, tot = O.sample_topk_np(vals, idx, temperature, u, fmt)
    np.testing.assert_allclose(probs, ep, rtol=PROB_RTOL, atol=PROB_ATOL, err_msg=what)
    for s in range(bits.shape[0]):
        m = int(np.sum(idx[s] >= 0))
        if m == 0:
            assert samples[s] == -1
            continue
        r = int(np.nonzero(idx[s] == samples[s])[0][0])
        target, tol = float(u[s]) * tot[s], SAMPLE_RTOL * tot[s]
        lo = cum[s, r - 1] if r > 0 else 0.0
        assert lo - tol <= target <= cum[s, r] + tol, (what, s, r)
        if np.min(np.abs(cum[s, :m] - target)) > tol:
            assert samples[s] == es[s], (what, s)
    return samples, probs


@pytest.mark.parametrize("temperature", [0.7, 1.0, 2.5])
def test_sample_llm_logits_full(temperature):
    bits = wl.llm_logits()
    rng = np.random.default_rng(int(temperature * 10))
    check_sample(bits, 50, temperature, rng.random(bits.shape[0]), "llm_logits")


def test_sample_bf16_logits():
    import torch

    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 32000)).astype(np.float32) * 2.0
    bits = torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)
    check_sample(bits, 40, 0.8, rng.random(64), "bf16 logits", fmt="bf16")


@pytest.mark.parametrize("k", [1, 7, 64, 65, 256, 1024])
def test_sample_k_sweep(k):
    rng = np.random.default_rng(k)
    bits = (rng.standard_normal((8, 5000)) * 2).astype(np.float16).view(np.uint16)
    check_sample(bits, k, 1.0, rng.random(8), f"k sweep {k}")


def test_sample_special_rows():
    rng = np.random.default_rng(8)
    rows = np.empty((6, 3000), dtype=np.uint16)
    rows[0] = 0xFC00                                        # all -inf: uniform over the top-k
    rows[1] = 0x7E00                                        # all NaN: rank 0 only
    rows[2] = (rng.standard_normal(3000)).astype(np.float16).view(np.uint16)
    rows[2, rng.integers(0, 3000, 5)] = 0x7C00              # a few +inf: shared among them
    rows[3] = np.float16(1.5).view(np.uint16)               # all equal
    rows[4] = (rng.standard_normal(3000)).astype(np.float16).view(np.uint16)
    rows[4, rng.random(3000) < 0.5] = 0x7E00                # half NaN
    rows[5] = (rng.integers(-4, 4, 3000) * 0.25).astype(np.float16).view(np.uint16)  # ties
    check_sample(rows, 50, 1.0, rng.random(6), "special rows")


def test_sample_histogram_on_uniform_grid():
    # One row replicated n times with u on a regular grid: the sampled-rank histogram must
    # equal n * probability (to within the rounding of the grid and fp32 boundaries).
    rng = np.random.default_rng(12)
    k, n = 32, 4096
    row = (rng.standard_normal(9000) * 1.5).astype(np.float16).view(np.uint16)
    bits = np.tile(row, (n, 1))
    u = (np.arange(n) + 0.5) / n
    samples, probs = check_sample(bits, k, 1.2, u, "uniform grid")
    _, idx = O.batch_topk_half(row[None, :], k, seg_len=row.size)
    rank_of = {int(i): r for r, i in enumerate(idx[0])}
    counts = np.bincount([rank_of[int(s)] for s in samples], minlength=k)
    assert np.all(np.abs(counts - n * probs[0]) <= 2.0)


def test_sample_without_probs_and_torch_convenience():
    import torch

    rng = np.random.default_rng(13)
    x = torch.from_numpy((rng.standard_normal((16, 7000)) * 2).astype(np.float16)).to("cuda:0")
    u = torch.from_numpy(rng.random(16).astype(np.float32)).to("cuda:0")
    announce("sample torch convenience 16x7000 k=20")
    samples, vals, idx, probs = bt.sample(x, 20, 0.9, u)
    torch.cuda.synchronize()
    assert probs is None
    bits = x.cpu().numpy().view(np.uint16)
    es, _, cum, tot = O.sample_topk_np(vals.cpu().view(torch.int16).numpy().view(np.uint16),
                                       idx.cpu().numpy(), 0.9, u.cpu().numpy())
    ev, ei = O.batch_topk_half(bits, 20, seg_len=7000)
    assert np.array_equal(idx.cpu().numpy(), ei)
    got = samples.cpu().numpy()
    for s in range(16):
        target = float(u[s]) * tot[s]
        if np.min(np.abs(cum[s, :20] - target)) > SAMPLE_RTOL * tot[s]:
            assert got[s] == es[s]


@pytest.mark.parametrize("seg_num,seg_len,k", [
    (3, 300_000, 50),     # several workgroups per row, the last one merges and samples
    (2, 600_000, 512),    # cooperative plan: the stand-alone sampling kernel follows
])
def test_sample_multi_workgroup_plans(seg_num, seg_len, k):
    rng = np.random.default_rng(seg_len + k)
    bits = (rng.standard_normal((seg_num, seg_len)) * 2).astype(np.float16).view(np.uint16)
    check_sample(bits, k, 1.0, rng.random(seg_num), f"multi-workgroup {seg_num}x{seg_len}")
