"""batch_topk for AMD Instinct MI355X (gfx950).

Python mirror of the reference host API (reference include/batch_topk.cuh:10-21) over the
C ABI of ``libbatch_topk_amd.so`` (declared in include/batch_topk.h).  The functions keep
the reference's names, argument order and meaning, and its error behaviour: they return a
hipError_t code (0 success, 1 = hipErrorInvalidValue for a rejected argument).  Pointers
are plain integers (device addresses); ``stream`` is a hipStream_t handle (0 = null stream).

``topk`` and ``segmented_topk`` are torch conveniences built on the same C ABI: torch
provides device memory and the stream, the HIP kernels do the work.  There is no CPU
fallback: if the library is missing every call raises.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# BATCH_TOPK_AMD_LIB selects another build of the same library (e.g. a tuning variant).
LIB_PATH = os.environ.get("BATCH_TOPK_AMD_LIB") or os.path.join(_HERE, "libbatch_topk_amd.so")

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1
MAX_K = 1024
PAD_INDEX = -1
PAD_VALUE_BITS = 0xFFFF

# Every extern "C" symbol declared in include/batch_topk.h.
EXPORTED_SYMBOLS = (
    "radix_topk_batch_topk_half",
    "radix_topk_batch_topk_half_workspace_size",
    "radix_topk_batch_topk_half_segmented",
    "radix_topk_batch_topk_half_segmented_workspace_size",
    "radix_topk_batch_topk_bf16",
    "radix_topk_batch_topk_bf16_workspace_size",
    "radix_topk_batch_topk_bf16_segmented",
    "radix_topk_batch_topk_bf16_segmented_workspace_size",
    "radix_topk_sample_half",
    "radix_topk_sample_half_workspace_size",
    "radix_topk_sample_bf16",
    "radix_topk_sample_bf16_workspace_size",
    "radix_topk_batch_topk_ex",
    "radix_topk_batch_topk_ex_workspace_size",
    "radix_topk_batch_topk_f32",
    "radix_topk_batch_topk_f32_workspace_size",
    "radix_topk_batch_topk_f32_segmented",
    "radix_topk_batch_topk_f32_segmented_workspace_size",
    "radix_topk_workspace_status",
    "radix_topk_debug_wait_hook",
    "radix_topk_batch_topk_half_noalloc",
)

# radix_topk_batch_topk_half_noalloc: its static per-GPU workspace (include/batch_topk.h)
NOALLOC_SCRATCH_BYTES = 8 << 20
HIP_ERROR_OUT_OF_MEMORY = 2

# radix_topk_workspace_status codes (include/batch_topk.h)
STATUS_OK = 0
STATUS_WAIT_TIMEOUT = 1

# radix_topk_batch_topk_ex element formats and output flags (include/batch_topk.h)
FORMAT_F16 = 0
FORMAT_BF16 = 1
FORMAT_F32 = 2
UNSORTED = 1
INDICES_ONLY = 2

_lib = None


class TopkError(RuntimeError):
    """A nonzero hipError_t returned by the engine."""

    def __init__(self, code: int, what: str):
        super().__init__(f"{what} failed with hipError_t {code}")
        self.code = code


def load_library():
    """Load the in-tree HIP engine; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP engine with `python -m batch_topk_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        vp, i32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        L.radix_topk_batch_topk_half.restype = i32
        L.radix_topk_batch_topk_half.argtypes = [vp, i32, i32, i32, vp, vp, vp, sz, vp]
        L.radix_topk_batch_topk_half_workspace_size.restype = sz
        L.radix_topk_batch_topk_half_workspace_size.argtypes = [i32, i32, i32]
        L.radix_topk_batch_topk_half_segmented.restype = i32
        L.radix_topk_batch_topk_half_segmented.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp, sz, vp]
        L.radix_topk_batch_topk_half_segmented_workspace_size.restype = sz
        L.radix_topk_batch_topk_half_segmented_workspace_size.argtypes = [i32, i32, i32]
        L.radix_topk_batch_topk_bf16.restype = i32
        L.radix_topk_batch_topk_bf16.argtypes = [vp, i32, i32, i32, vp, vp, vp, sz, vp]
        L.radix_topk_batch_topk_bf16_workspace_size.restype = sz
        L.radix_topk_batch_topk_bf16_workspace_size.argtypes = [i32, i32, i32]
        L.radix_topk_batch_topk_bf16_segmented.restype = i32
        L.radix_topk_batch_topk_bf16_segmented.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp, sz, vp]
        L.radix_topk_batch_topk_bf16_segmented_workspace_size.restype = sz
        L.radix_topk_batch_topk_bf16_segmented_workspace_size.argtypes = [i32, i32, i32]
        f32 = ctypes.c_float
        for name in ("radix_topk_sample_half", "radix_topk_sample_bf16"):
            fn = getattr(L, name)
            fn.restype = i32
            fn.argtypes = [vp, i32, i32, i32, f32, vp, vp, vp, vp, vp, vp, sz, vp]
            ws = getattr(L, name + "_workspace_size")
            ws.restype = sz
            ws.argtypes = [i32, i32, i32]
        L.radix_topk_batch_topk_f32.restype = i32
        L.radix_topk_batch_topk_f32.argtypes = [vp, i32, i32, i32, vp, vp, vp, sz, vp]
        L.radix_topk_batch_topk_f32_workspace_size.restype = sz
        L.radix_topk_batch_topk_f32_workspace_size.argtypes = [i32, i32, i32]
        L.radix_topk_batch_topk_f32_segmented.restype = i32
        L.radix_topk_batch_topk_f32_segmented.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp, sz, vp]
        L.radix_topk_batch_topk_f32_segmented_workspace_size.restype = sz
        L.radix_topk_batch_topk_f32_segmented_workspace_size.argtypes = [i32, i32, i32]
        L.radix_topk_batch_topk_ex.restype = i32
        L.radix_topk_batch_topk_ex.argtypes = [vp, i32, vp, i32, i32, i32, i32, vp, vp, vp, sz, vp]
        L.radix_topk_batch_topk_ex_workspace_size.restype = sz
        L.radix_topk_batch_topk_ex_workspace_size.argtypes = [i32, i32, i32, i32, i32]
        L.radix_topk_workspace_status.restype = i32
        L.radix_topk_workspace_status.argtypes = [vp, sz, i32, vp, vp]
        L.radix_topk_batch_topk_half_noalloc.restype = i32
        L.radix_topk_batch_topk_half_noalloc.argtypes = [vp, i32, i32, i32, vp, vp, vp]
        L.radix_topk_debug_wait_hook.restype = None
        L.radix_topk_debug_wait_hook.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        _lib = L
    return _lib


# ------------------------------------------------------------------ reference-shaped API

def batch_topk_half(d_input: int, seg_num: int, seg_len: int, k: int, d_output_values: int,
                    d_output_indices: int, d_workspace: int, workspace_bytes: int,
                    stream: int = 0) -> int:
    """reference include/batch_topk.cuh:10-19 -> hipError_t code."""
    return int(load_library().radix_topk_batch_topk_half(
        d_input, seg_num, seg_len, k, d_output_values, d_output_indices, d_workspace,
        workspace_bytes, stream))


def batch_topk_half_noalloc(d_input: int, seg_num: int, seg_len: int, k: int, d_output_values: int,
                            d_output_indices: int, stream: int = 0) -> int:
    """radix_topk_batch_topk_half_noalloc: batch_topk_half with the library's static per-GPU
    workspace (no workspace argument, nothing allocated) -> hipError_t code."""
    return int(load_library().radix_topk_batch_topk_half_noalloc(
        d_input, seg_num, seg_len, k, d_output_values, d_output_indices, stream))


def batch_topk_half_workspace_size(seg_num: int, seg_len: int, k: int) -> int:
    """reference include/batch_topk.cuh:21 -> bytes (0 for an unsupported shape)."""
    return int(load_library().radix_topk_batch_topk_half_workspace_size(seg_num, seg_len, k))


def batch_topk_half_segmented(d_input: int, d_offsets: int, seg_num: int, max_seg_len: int,
                              k: int, d_output_values: int, d_output_indices: int,
                              d_workspace: int, workspace_bytes: int, stream: int = 0) -> int:
    """Variable-length segments given by a device int32 offset array -> hipError_t code."""
    return int(load_library().radix_topk_batch_topk_half_segmented(
        d_input, d_offsets, seg_num, max_seg_len, k, d_output_values, d_output_indices,
        d_workspace, workspace_bytes, stream))


def batch_topk_half_segmented_workspace_size(seg_num: int, max_seg_len: int, k: int) -> int:
    return int(load_library().radix_topk_batch_topk_half_segmented_workspace_size(
        seg_num, max_seg_len, k))


def batch_topk_bf16(d_input: int, seg_num: int, seg_len: int, k: int, d_output_values: int,
                    d_output_indices: int, d_workspace: int, workspace_bytes: int,
                    stream: int = 0) -> int:
    """bfloat16 twin of batch_topk_half (same arguments and contract) -> hipError_t code."""
    return int(load_library().radix_topk_batch_topk_bf16(
        d_input, seg_num, seg_len, k, d_output_values, d_output_indices, d_workspace,
        workspace_bytes, stream))


def batch_topk_bf16_workspace_size(seg_num: int, seg_len: int, k: int) -> int:
    return int(load_library().radix_topk_batch_topk_bf16_workspace_size(seg_num, seg_len, k))


def batch_topk_bf16_segmented(d_input: int, d_offsets: int, seg_num: int, max_seg_len: int,
                              k: int, d_output_values: int, d_output_indices: int,
                              d_workspace: int, workspace_bytes: int, stream: int = 0) -> int:
    """bfloat16 twin of batch_topk_half_segmented -> hipError_t code."""
    return int(load_library().radix_topk_batch_topk_bf16_segmented(
        d_input, d_offsets, seg_num, max_seg_len, k, d_output_values, d_output_indices,
        d_workspace, workspace_bytes, stream))


def batch_topk_bf16_segmented_workspace_size(seg_num: int, max_seg_len: int, k: int) -> int:
    return int(load_library().radix_topk_batch_topk_bf16_segmented_workspace_size(
        seg_num, max_seg_len, k))


def sample_half(d_logits: int, seg_num: int, seg_len: int, k: int, temperature: float,
                d_uniforms: int, d_topk_values: int, d_topk_indices: int, d_probs: int,
                d_samples: int, d_workspace: int, workspace_bytes: int, stream: int = 0) -> int:
    """Top-k sampling over fp16 logits (include/batch_topk.h) -> hipError_t code.
    ``d_probs`` may be 0 (no probabilities written)."""
    return int(load_library().radix_topk_sample_half(
        d_logits, seg_num, seg_len, k, float(temperature), d_uniforms, d_topk_values,
        d_topk_indices, d_probs or None, d_samples, d_workspace, workspace_bytes, stream))


def sample_half_workspace_size(seg_num: int, seg_len: int, k: int) -> int:
    return int(load_library().radix_topk_sample_half_workspace_size(seg_num, seg_len, k))


def sample_bf16(d_logits: int, seg_num: int, seg_len: int, k: int, temperature: float,
                d_uniforms: int, d_topk_values: int, d_topk_indices: int, d_probs: int,
                d_samples: int, d_workspace: int, workspace_bytes: int, stream: int = 0) -> int:
    """Top-k sampling over bfloat16 logits -> hipError_t code."""
    return int(load_library().radix_topk_sample_bf16(
        d_logits, seg_num, seg_len, k, float(temperature), d_uniforms, d_topk_values,
        d_topk_indices, d_probs or None, d_samples, d_workspace, workspace_bytes, stream))


def sample_bf16_workspace_size(seg_num: int, seg_len: int, k: int) -> int:
    return int(load_library().radix_topk_sample_bf16_workspace_size(seg_num, seg_len, k))


def batch_topk_f32(d_input: int, seg_num: int, seg_len: int, k: int, d_output_values: int,
                   d_output_indices: int, d_workspace: int, workspace_bytes: int,
                   stream: int = 0) -> int:
    """radix_topk_batch_topk_f32: fixed-length rows of float (values out as float bits)."""
    return int(load_library().radix_topk_batch_topk_f32(
        d_input, seg_num, seg_len, k, d_output_values, d_output_indices, d_workspace,
        workspace_bytes, stream))


def batch_topk_f32_workspace_size(seg_num: int, seg_len: int, k: int) -> int:
    return int(load_library().radix_topk_batch_topk_f32_workspace_size(seg_num, seg_len, k))


def batch_topk_f32_segmented(d_input: int, d_offsets: int, seg_num: int, max_seg_len: int,
                             k: int, d_output_values: int, d_output_indices: int,
                             d_workspace: int, workspace_bytes: int, stream: int = 0) -> int:
    return int(load_library().radix_topk_batch_topk_f32_segmented(
        d_input, d_offsets, seg_num, max_seg_len, k, d_output_values, d_output_indices,
        d_workspace, workspace_bytes, stream))


def batch_topk_f32_segmented_workspace_size(seg_num: int, max_seg_len: int, k: int) -> int:
    return int(load_library().radix_topk_batch_topk_f32_segmented_workspace_size(seg_num, max_seg_len, k))


def batch_topk_ex(d_input: int, fmt: int, d_offsets: int, seg_num: int, seg_len: int, k: int,
                  flags: int, d_output_values: int, d_output_indices: int, d_workspace: int,
                  workspace_bytes: int, stream: int = 0) -> int:
    """radix_topk_batch_topk_ex (include/batch_topk.h): any layout (d_offsets 0 = fixed
    length), format (FORMAT_F16 / FORMAT_BF16) and output flags (UNSORTED, INDICES_ONLY)."""
    return int(load_library().radix_topk_batch_topk_ex(
        d_input, fmt, d_offsets or None, seg_num, seg_len, k, flags, d_output_values or None,
        d_output_indices, d_workspace, workspace_bytes, stream))


def batch_topk_ex_workspace_size(fmt: int, segmented: bool, seg_num: int, seg_len: int, k: int) -> int:
    return int(load_library().radix_topk_batch_topk_ex_workspace_size(fmt, int(bool(segmented)),
                                                                      seg_num, seg_len, k))


def workspace_status(d_workspace: int, workspace_bytes: int, seg_num: int, stream: int = 0):
    """radix_topk_workspace_status: per-segment status words of the last call made with the
    workspace (STATUS_OK or STATUS_WAIT_TIMEOUT), as a list; synchronises ``stream``."""
    buf = (ctypes.c_uint32 * max(1, seg_num))()
    rc = int(load_library().radix_topk_workspace_status(d_workspace, workspace_bytes, seg_num, buf, stream))
    if rc != HIP_SUCCESS:
        raise TopkError(rc, "radix_topk_workspace_status")
    return [int(v) for v in buf[:seg_num]]


def debug_wait_hook(spin_limit: int, force_mask: int = 0) -> None:
    """radix_topk_debug_wait_hook (test hook): bound every cross-workgroup wait at spin_limit
    polls and force the waits named by force_mask to time out; (0, 0) restores ordinary calls."""
    load_library().radix_topk_debug_wait_hook(spin_limit, force_mask)


# ------------------------------------------------------------------ torch conveniences

def _entry_points(dtype):
    """(fixed, fixed workspace, segmented, segmented workspace) for a torch dtype."""
    import torch

    if dtype == torch.float16:
        return (batch_topk_half, batch_topk_half_workspace_size, batch_topk_half_segmented,
                batch_topk_half_segmented_workspace_size)
    if dtype == torch.bfloat16:
        return (batch_topk_bf16, batch_topk_bf16_workspace_size, batch_topk_bf16_segmented,
                batch_topk_bf16_segmented_workspace_size)
    if dtype == torch.float32:
        return (batch_topk_f32, batch_topk_f32_workspace_size, batch_topk_f32_segmented,
                batch_topk_f32_segmented_workspace_size)
    raise ValueError(f"unsupported dtype {dtype}: float16, bfloat16 or float32")


def _on_stream(stream):
    """Makes ``stream`` current while a call allocates its outputs and temporary workspace, so
    that torch's caching allocator ties them to the stream the kernel runs on (a temporary freed
    on return is then reused only by work ordered after the kernel)."""
    import contextlib

    import torch

    return torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()


def _stream_handle(stream) -> int:
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _format_of(dtype) -> int:
    import torch

    if dtype == torch.float16:
        return FORMAT_F16
    if dtype == torch.bfloat16:
        return FORMAT_BF16
    if dtype == torch.float32:
        return FORMAT_F32
    raise ValueError(f"unsupported dtype {dtype}: float16, bfloat16 or float32")


def _topk_ex(x, offsets, seg_num, seg_len, k, sorted, values, workspace, stream):
    import torch

    fmt = _format_of(x.dtype)
    flags = (0 if sorted else UNSORTED) | (0 if values else INDICES_ONLY)
    ws_bytes = batch_topk_ex_workspace_size(fmt, offsets is not None, seg_num, seg_len, k)
    if ws_bytes == 0:
        raise TopkError(HIP_ERROR_INVALID_VALUE, "radix_topk_batch_topk_ex_workspace_size")
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    vals = torch.empty((seg_num, k), dtype=x.dtype, device=x.device) if values else None
    idx = torch.empty((seg_num, k), dtype=torch.int32, device=x.device)
    rc = batch_topk_ex(x.data_ptr(), fmt, offsets.data_ptr() if offsets is not None else 0, seg_num,
                       seg_len, k, flags, vals.data_ptr() if values else 0, idx.data_ptr(),
                       workspace.data_ptr(), workspace.numel(), _stream_handle(stream))
    if rc != HIP_SUCCESS:
        raise TopkError(rc, "radix_topk_batch_topk_ex")
    return vals, idx


def topk(x, k: int, workspace=None, stream=None, sorted: bool = True, values: bool = True):
    """Top-k of every row of a contiguous float16, bfloat16 or float32 CUDA tensor [seg_num, seg_len].

    Returns (values [seg_num, k] of x's dtype, indices int32 [seg_num, k]).  ``workspace``
    may be a uint8 CUDA tensor of at least the workspace size of the shape.  ``sorted=False``
    returns each row's top-k in unspecified order; ``values=False`` returns (None, indices).
    ``stream`` (a torch.cuda.Stream, default the current one) runs the kernel; the outputs are
    allocated on it.
    """
    with _on_stream(stream):
        return _topk(x, k, workspace, stream, sorted, values)


def _topk(x, k, workspace, stream, sorted, values):
    import torch

    if x.dim() != 2 or not x.is_cuda or not x.is_contiguous():
        raise ValueError("topk expects a contiguous 2-D float16, bfloat16 or float32 CUDA tensor")
    if not (sorted and values):
        return _topk_ex(x, None, x.shape[0], x.shape[1], k, sorted, values, workspace, stream)
    fixed, fixed_ws, _, _ = _entry_points(x.dtype)
    seg_num, seg_len = x.shape
    ws_bytes = fixed_ws(seg_num, seg_len, k)
    if ws_bytes == 0:
        raise TopkError(HIP_ERROR_INVALID_VALUE, f"{fixed.__name__}_workspace_size")
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    vals = torch.empty((seg_num, k), dtype=x.dtype, device=x.device)
    idx = torch.empty((seg_num, k), dtype=torch.int32, device=x.device)
    rc = fixed(x.data_ptr(), seg_num, seg_len, k, vals.data_ptr(), idx.data_ptr(),
               workspace.data_ptr(), workspace.numel(), _stream_handle(stream))
    if rc != HIP_SUCCESS:
        raise TopkError(rc, fixed.__name__)
    return vals, idx


def segmented_topk(x, offsets, k: int, max_seg_len: int, workspace=None, stream=None,
                   sorted: bool = True, values: bool = True):
    """Top-k of every segment x[offsets[s]:offsets[s+1]] of a 1-D float16, bfloat16 or float32
    CUDA tensor.

    ``offsets`` is an int32 CUDA tensor of seg_num + 1 entries.  Ranks beyond a segment's
    length hold index -1 and value bits 0xFFFF.  ``sorted``, ``values`` and ``stream`` as for
    topk.
    """
    with _on_stream(stream):
        return _segmented_topk(x, offsets, k, max_seg_len, workspace, stream, sorted, values)


def _segmented_topk(x, offsets, k, max_seg_len, workspace, stream, sorted, values):
    import torch

    if not x.is_cuda or not x.is_contiguous():
        raise ValueError("segmented_topk expects a contiguous float16, bfloat16 or float32 CUDA tensor")
    if offsets.dtype != torch.int32 or not offsets.is_cuda or offsets.dim() != 1:
        raise ValueError("offsets must be a 1-D int32 CUDA tensor")
    if not (sorted and values):
        return _topk_ex(x, offsets, offsets.numel() - 1, max_seg_len, k, sorted, values,
                        workspace, stream)
    _, _, seg, seg_ws = _entry_points(x.dtype)
    seg_num = offsets.numel() - 1
    ws_bytes = seg_ws(seg_num, max_seg_len, k)
    if ws_bytes == 0:
        raise TopkError(HIP_ERROR_INVALID_VALUE, f"{seg.__name__}_workspace_size")
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    vals = torch.empty((seg_num, k), dtype=x.dtype, device=x.device)
    idx = torch.empty((seg_num, k), dtype=torch.int32, device=x.device)
    rc = seg(x.data_ptr(), offsets.data_ptr(), seg_num, max_seg_len, k, vals.data_ptr(),
             idx.data_ptr(), workspace.data_ptr(), workspace.numel(), _stream_handle(stream))
    if rc != HIP_SUCCESS:
        raise TopkError(rc, seg.__name__)
    return vals, idx


def sample(logits, k: int, temperature: float, uniforms, with_probs: bool = False,
           workspace=None, stream=None):
    """Top-k sampling: one index per row of a contiguous float16 / bfloat16 CUDA tensor
    [seg_num, seg_len] of logits, drawn from the softmax of the row's top-k at
    ``temperature`` with ``uniforms`` (float32 CUDA tensor [seg_num], values in [0, 1)).

    Returns (samples int32 [seg_num], top-k values, top-k indices, probs float32
    [seg_num, k] or None).  ``stream`` as for topk.
    """
    with _on_stream(stream):
        return _sample(logits, k, temperature, uniforms, with_probs, workspace, stream)


def _sample(logits, k, temperature, uniforms, with_probs, workspace, stream):
    import torch

    if logits.dim() != 2 or not logits.is_cuda or not logits.is_contiguous():
        raise ValueError("sample expects a contiguous 2-D float16 or bfloat16 CUDA tensor")
    if uniforms.dtype != torch.float32 or not uniforms.is_cuda or uniforms.numel() != logits.shape[0]:
        raise ValueError("uniforms must be a float32 CUDA tensor with one entry per row")
    if logits.dtype == torch.float16:
        fn, ws_size = sample_half, sample_half_workspace_size
    elif logits.dtype == torch.bfloat16:
        fn, ws_size = sample_bf16, sample_bf16_workspace_size
    else:
        raise ValueError(f"unsupported dtype {logits.dtype}: float16 or bfloat16")
    seg_num, seg_len = logits.shape
    ws_bytes = ws_size(seg_num, seg_len, k)
    if ws_bytes == 0:
        raise TopkError(HIP_ERROR_INVALID_VALUE, f"{fn.__name__}_workspace_size")
    if workspace is None:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=logits.device)
    vals = torch.empty((seg_num, k), dtype=logits.dtype, device=logits.device)
    idx = torch.empty((seg_num, k), dtype=torch.int32, device=logits.device)
    probs = torch.empty((seg_num, k), dtype=torch.float32, device=logits.device) if with_probs else None
    samples = torch.empty(seg_num, dtype=torch.int32, device=logits.device)
    rc = fn(logits.data_ptr(), seg_num, seg_len, k, temperature, uniforms.data_ptr(), vals.data_ptr(),
            idx.data_ptr(), probs.data_ptr() if probs is not None else 0, samples.data_ptr(),
            workspace.data_ptr(), workspace.numel(), _stream_handle(stream))
    if rc != HIP_SUCCESS:
        raise TopkError(rc, fn.__name__)
    return samples, vals, idx, probs
