"""Helpers for the GPU parity tests: every call goes through the C ABI (include/batch_topk.h)
with device buffers that torch allocates; results come back as raw fp16 bits + int32."""

from __future__ import annotations

import sys

import numpy as np

import batch_topk_amd as bt


def announce(msg: str) -> None:
    """Name the case on stdout before a GPU step (visible even if the step takes the box down)."""
    sys.stdout.write(f"[gpu-case] {msg}\n")
    sys.stdout.flush()


def _torch():
    import torch

    return torch


def device_u16(bits: np.ndarray, pad_front: int = 0, pad_back: int = 8):
    torch = _torch()
    flat = np.ascontiguousarray(bits, dtype=np.uint16).reshape(-1)
    host = np.full(flat.size + pad_front + pad_back, 0x7E00, dtype=np.uint16)
    host[pad_front:pad_front + flat.size] = flat
    return torch.from_numpy(host.view(np.int16)).to("cuda:0")


def run_fixed(bits: np.ndarray, k: int, poison: int | None = None, elem_offset: int = 0,
              workspace=None, expect_rc: int = 0, fmt: str = "f16"):
    """radix_topk_batch_topk_{half,bf16} on [seg_num, seg_len] bits -> (values u16, indices i32)."""
    torch = _torch()
    seg_num, seg_len = bits.shape
    buf = device_u16(bits, pad_front=elem_offset)
    call, ws_size = ((bt.batch_topk_half, bt.batch_topk_half_workspace_size) if fmt == "f16"
                     else (bt.batch_topk_bf16, bt.batch_topk_bf16_workspace_size))
    ws_bytes = ws_size(seg_num, seg_len, k)
    assert ws_bytes > 0, (seg_num, seg_len, k)
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
        if poison is not None:
            workspace.fill_(poison)
    vals = torch.full((seg_num, k), 0x1234, dtype=torch.int16, device="cuda:0")
    idx = torch.full((seg_num, k), -7, dtype=torch.int32, device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    rc = call(buf.data_ptr() + 2 * elem_offset, seg_num, seg_len, k,
              vals.data_ptr(), idx.data_ptr(), workspace.data_ptr(), ws_bytes, stream)
    assert rc == expect_rc
    torch.cuda.synchronize()
    return vals.cpu().numpy().view(np.uint16), idx.cpu().numpy()


def run_segmented(bits: np.ndarray, offsets: np.ndarray, k: int, max_seg_len: int,
                  poison: int | None = None, elem_offset: int = 0, fmt: str = "f16"):
    torch = _torch()
    seg_num = offsets.size - 1
    buf = device_u16(bits, pad_front=elem_offset)
    off = torch.from_numpy(np.ascontiguousarray(offsets, dtype=np.int32)).to("cuda:0")
    call, ws_size = ((bt.batch_topk_half_segmented, bt.batch_topk_half_segmented_workspace_size)
                     if fmt == "f16" else
                     (bt.batch_topk_bf16_segmented, bt.batch_topk_bf16_segmented_workspace_size))
    ws_bytes = ws_size(seg_num, max_seg_len, k)
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
    if poison is not None:
        ws.fill_(poison)
    vals = torch.full((seg_num, k), 0x1234, dtype=torch.int16, device="cuda:0")
    idx = torch.full((seg_num, k), -7, dtype=torch.int32, device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    rc = call(buf.data_ptr() + 2 * elem_offset, off.data_ptr(), seg_num, max_seg_len, k,
              vals.data_ptr(), idx.data_ptr(), ws.data_ptr(), ws_bytes, stream)
    assert rc == 0
    torch.cuda.synchronize()
    return vals.cpu().numpy().view(np.uint16), idx.cpu().numpy()


def assert_same(got, exp, what: str):
    gv, gi = got
    ev, ei = exp
    if not np.array_equal(gi, ei) or not np.array_equal(gv, ev):
        bad = np.argwhere((gi != ei) | (gv != ev))
        s, r = bad[0]
        raise AssertionError(
            f"{what}: {len(bad)} mismatching ranks; first at segment {s} rank {r}: "
            f"got (idx {gi[s, r]}, bits {gv[s, r]:#06x}) expected (idx {ei[s, r]}, bits {ev[s, r]:#06x})")


def assert_properties(bits_rows, vals, idx, k, lengths, fmt: str = "f16"):
    """Size-independent invariants: indices in range and unique, values equal the input at
    the index, keys non-decreasing with ascending index inside equal keys, pads after len."""
    from oracle.oracle import encode_bf16_desc_np, encode_half_desc_np  # checker only

    if fmt != "f16":
        encode_half_desc_np = encode_bf16_desc_np  # noqa: F811 (same statement, bf16 key)

    for s, row in enumerate(bits_rows):
        n = lengths[s]
        m = min(k, n)
        ii = idx[s, :m]
        assert np.all((ii >= 0) & (ii < n)), s
        assert np.unique(ii).size == m, s
        assert np.array_equal(vals[s, :m], row[ii]), s
        kk = encode_half_desc_np(row[ii]).astype(np.int64)
        comp = kk * (1 << 32) + ii
        assert np.all(np.diff(comp) > 0), s
        assert np.all(idx[s, m:] == -1) and np.all(vals[s, m:] == 0xFFFF), s
        if m < n:
            # every unselected key is >= the last selected key
            all_keys = encode_half_desc_np(row).astype(np.int64)
            assert np.sum(all_keys < kk[-1]) <= m - 1, s
