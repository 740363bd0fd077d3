"""Compile the HIP engine into batch_topk_amd/libbatch_topk_amd.so (gfx950 only).

Run as ``python -m batch_topk_amd.build``; ``__graft_entry__.build()`` calls ``build()``.
The library is built in-tree so that it travels with the source tree.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libbatch_topk_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

SOURCES = ["topk_kernels.hip", "sample_kernels.hip", "noalloc.hip", "api.cpp"]
# Measurement reference (not part of the engine): the single-pass read floor, loaded by
# batch_topk_amd/profiling.py only.
FLOOR_LIB_PATH = os.path.join(HERE, "libread_floor.so")
FLOOR_SOURCES = ["read_floor.hip"]
# A C++ caller of the reference's host API compiled against include/batch_topk.hpp and linked
# against the engine (run by tests/test_cpp_dropin_gpu.py).
ROOT = os.path.dirname(HERE)
CPP_CALLER_SRC = os.path.join(ROOT, "tests", "cpp", "dropin_caller.cpp")
CPP_CALLER_BIN = os.path.join(ROOT, "tests", "cpp", "dropin_caller")
# Measurement build of the engine with the per-phase clock stamps compiled in
# (-DTOPK_PHASE_TRACE): loaded by batch_topk_amd/profiling.py only, never by the package.
TRACE_LIB_PATH = os.path.join(HERE, "libbatch_topk_amd_trace.so")

# -packed-fp32-ops: no v_pk_*_f32 in any code object (this engine has no fp32 math anyway).
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP engine cannot be built")
    return path


def _run(cmd, verbose: bool, what: str) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed to build " + what)


def _object(source: str, out_dir: str, verbose: bool, defines=()) -> str:
    """One translation unit compiled to an object (host code and its gfx950 device code)."""
    tag = "_".join(d.lower() for d in defines)
    obj = os.path.join(out_dir, os.path.splitext(source)[0] + (("." + tag) if tag else "") + ".o")
    _run([hipcc(), *HIP_FLAGS, *[f"-D{d}" for d in defines], "-c", "-o", obj, os.path.join(CSRC, source)],
         verbose, source)
    return obj


def _link(objects, out_path: str, verbose: bool) -> None:
    tmp = out_path + ".tmp"
    _run([hipcc(), *HIP_FLAGS, "-shared", "-o", tmp, *objects, "-lamdhip64"], verbose,
         os.path.basename(out_path))
    os.replace(tmp, out_path)


def build_cpp_caller(verbose: bool = False) -> str:
    """The drop-in C++ caller (host code only), linked against the in-tree engine library."""
    tmp = CPP_CALLER_BIN + ".tmp"
    cmd = [hipcc(), "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"), "-o", tmp,
           CPP_CALLER_SRC, "-L", HERE, "-lbatch_topk_amd", "-Wl,-rpath,$ORIGIN/../../batch_topk_amd"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed to build the drop-in C++ caller")
    os.replace(tmp, CPP_CALLER_BIN)
    return CPP_CALLER_BIN


def build(verbose: bool = False) -> str:
    """Always recompiles (the build check must exercise the compiler): the engine library, the
    two measurement libraries (read floor, phase-traced engine) and the drop-in C++ caller.
    The translation units compile in parallel into a temporary directory, then link."""
    jobs = [(src, ()) for src in SOURCES] + [("topk_kernels.hip", ("TOPK_PHASE_TRACE",))]
    jobs += [(src, ()) for src in FLOOR_SOURCES]
    with tempfile.TemporaryDirectory(prefix="batch_topk_amd_build_") as out_dir:
        with concurrent.futures.ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1)) as pool:
            futures = [pool.submit(_object, src, out_dir, verbose, defs) for src, defs in jobs]
            objs = [f.result() for f in futures]
        engine = objs[:len(SOURCES)]
        trace = [objs[len(SOURCES)] if src == "topk_kernels.hip" else o for src, o in zip(SOURCES, engine)]
        floor = objs[len(SOURCES) + 1:]
        _link(engine, LIB_PATH, verbose)
        _link(trace, TRACE_LIB_PATH, verbose)
        _link(floor, FLOOR_LIB_PATH, verbose)
    build_cpp_caller(verbose)
    return LIB_PATH


def resource_usage(source: str = "topk_kernels.hip") -> dict:
    """Per-kernel VGPRs, scratch bytes per lane and occupancy (waves per SIMD) of the device
    code, from the compiler's kernel-resource-usage remarks (device-only compile)."""
    cmd = [hipcc(), *HIP_FLAGS, "--cuda-device-only", "-c", "-o", os.devnull,
           "-Rpass-analysis=kernel-resource-usage", os.path.join(CSRC, source)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed on the resource-usage compile")
    out: dict = {}
    name = None
    for line in res.stderr.splitlines():
        if "remark:" not in line:
            continue
        text = line.split("remark:", 1)[1].strip()
        text = text.replace("[-Rpass-analysis=kernel-resource-usage]", "").strip()
        if text.startswith("Function Name:"):
            name = text.split(":", 1)[1].strip()
            out[name] = {}
        elif name is not None and ":" in text:
            key, val = text.split(":", 1)
            val = val.strip()
            try:
                out[name][key.strip()] = int(val)
            except ValueError:
                out[name][key.strip()] = val
    return out


if __name__ == "__main__":
    print(build(verbose=True))
