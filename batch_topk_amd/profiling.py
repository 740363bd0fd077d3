"""Helpers for the rocprofv3 measurements of the engine (run on the GPU host).

  python -m batch_topk_amd.profiling copy [--mib 256] [--reps 5]
      Elementwise int16 copy of a buffer of known size (reads and writes MIB MiB per
      dispatch): the calibration kernel for the FETCH_SIZE / WRITE_SIZE counters.

  python -m batch_topk_amd.profiling counters DIR SUBSTRING
      Mean per dispatch of every counter in rocprofv3's counter_collection CSVs under DIR, for
      kernels whose name contains SUBSTRING.

  python -m batch_topk_amd.profiling stats DIR
      The kernel_stats CSV rocprofv3 --stats wrote under DIR, as a text table.

  python -m batch_topk_amd.profiling traffic --workload W --k K --kernel-fetch DIR
        --kernel-write DIR --copy-fetch DIR --copy-write DIR [--copy-mib 256] [--out FILE]
      HBM bytes per launch of the top-k kernel: its FETCH_SIZE and WRITE_SIZE (KiB per
      dispatch), each scaled by known bytes / measured KiB of the copy kernel, merged into the
      JSON table bench.py reads.

  python -m batch_topk_amd.profiling floor [--calls 2000]
      Back-to-back time of the single-pass read floor (libread_floor.so) over the 128 x 128,256
      fp16 batch, rotating over 17 input copies (557 MB), for several workgroup shapes.

  python -m batch_topk_amd.profiling matrix [--out FILE]
      bench.py over every workload (fp16; bf16 and the sampling consumer on the LLM logits;
      fp32 on every workload; the unsorted and indices-only outputs), as a markdown table.
"""

from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import os
import sys

KERNEL_SUBSTRING = "segmented_topk_kernel"
COPY_SUBSTRING = "CUDAFunctorOnSelf_add"


def counter_means(root: str, substring: str) -> dict:
    acc = collections.defaultdict(list)
    for path in glob.glob(os.path.join(root, "**", "*counter_collection.csv"), recursive=True):
        with open(path) as f:
            for row in csv.DictReader(f):
                if substring in row.get("Kernel_Name", ""):
                    acc[row["Counter_Name"]].append(float(row["Counter_Value"]))
    return {name: (sum(v) / len(v), len(v)) for name, v in acc.items()}


def kernel_stats(root: str) -> list:
    rows = []
    for path in glob.glob(os.path.join(root, "**", "*kernel_stats.csv"), recursive=True):
        with open(path) as f:
            rows.extend(csv.DictReader(f))
    return rows


def run_copy(mib: int, reps: int) -> None:
    import torch

    n = mib * 2**20 // 2
    src = torch.arange(n, dtype=torch.int16, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.add(src, 1, out=dst)
    torch.cuda.synchronize()
    print(f"copy: {reps} dispatches reading and writing {mib} MiB each")


FLOOR_SHAPES = ((1024, 16, 1), (512, 32, 1), (512, 16, 2), (1024, 8, 2), (256, 16, 4))


def run_floor(calls: int) -> None:
    import ctypes

    import numpy as np
    import torch

    from batch_topk_amd import build, workloads

    lib = ctypes.CDLL(build.FLOOR_LIB_PATH)
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    lib.read_floor_run.restype = i32
    lib.read_floor_run.argtypes = [vp, i32, i32, i32, i32, i32, i32, vp, vp]
    bits = workloads.llm_logits()
    rows, row_len = bits.shape
    src = torch.from_numpy(bits.view(np.int16)).to("cuda:0")
    copies = [src] + [src.clone() for _ in range(16)]
    ptrs = (ctypes.c_void_p * calls)(*[copies[i % len(copies)].data_ptr() for i in range(calls)])
    out = torch.empty(rows * 4 * 16, dtype=torch.int32, device="cuda:0")
    stream = torch.cuda.current_stream()
    nbytes = 2 * rows * row_len
    print(f"single-pass read of {rows} x {row_len} fp16 ({nbytes} bytes), {calls} back-to-back "
          f"launches over {len(copies)} input copies")
    lib.read_floor_empty_run.restype = i32
    lib.read_floor_empty_run.argtypes = [i32, i32, vp, vp]
    lib.read_floor_empty_run(calls, rows, out.data_ptr(), stream.cuda_stream)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    lib.read_floor_empty_run(calls, rows, out.data_ptr(), stream.cuda_stream)
    b.record(stream)
    torch.cuda.synchronize()
    print(f"empty kernel, {rows} workgroups x 1024 threads: {a.elapsed_time(b) * 1e3 / calls:.2f} us per launch")
    print("workgroups per row | threads x vectors | us per launch | GB/s | fraction of 8 TB/s")
    for block, vpt, w in FLOOR_SHAPES:
        def go():
            rc = lib.read_floor_run(ptrs, calls, rows, row_len, block, vpt, w, out.data_ptr(),
                                    stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"read_floor_run returned {rc}")
        go()  # warm-up
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        go()
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / calls
        print(f"{w} | {block} x {vpt} | {us:.2f} | {nbytes / us / 1e3:.0f} | {nbytes / us / 1e3 / 8000:.3f}")


MATRIX = (
    ("llm_logits", ["--k", "50"]),
    ("uniform_small", ["--k", "50"]),
    ("varlen", ["--k", "64"]),
    ("ties_special", ["--k", "1"]),
    ("ties_special", ["--k", "16"]),
    ("ties_special", ["--k", "128"]),
    ("ties_special", ["--k", "256"]),
    ("huge_segment", ["--k", "1024"]),
    ("llm_logits", ["--k", "50", "--dtype", "bf16"]),
    ("llm_logits", ["--k", "50", "--op", "sample"]),
    ("llm_logits", ["--k", "50", "--dtype", "f32"]),
    ("uniform_small", ["--k", "50", "--dtype", "f32"]),
    ("varlen", ["--k", "64", "--dtype", "f32"]),
    ("ties_special", ["--k", "16", "--dtype", "f32"]),
    ("ties_special", ["--k", "256", "--dtype", "f32"]),
    ("huge_segment", ["--k", "1024", "--dtype", "f32"]),
    ("ties_special", ["--k", "128", "--output", "unsorted"]),
    ("ties_special", ["--k", "256", "--output", "unsorted"]),
    ("varlen", ["--k", "64", "--output", "unsorted"]),
    ("llm_logits", ["--k", "50", "--output", "indices"]),
) + tuple(("ref_matrix", ["--k", "50", "--seg-num", str(n), "--no-cpu-baseline"])
          for n in (128, 1500, 3000, 4500, 6000))


def run_matrix(out_path) -> None:
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    lines = ["| workload | options | us per step | segments/s | elements/s | roofline frac | "
             "CPU 1 thread (segments/s) | CPU threaded | parity |", "|---|---|---|---|---|---|---|---|---|"]
    for workload, opts in MATRIX:
        cmd = [sys.executable, os.path.join(root, "bench.py"), "--workload", workload, *opts]
        res = subprocess.run(cmd, capture_output=True, text=True, cwd=root)
        if res.returncode != 0:
            sys.stderr.write(res.stderr)
            raise RuntimeError("bench.py failed: " + " ".join(cmd))
        d = json.loads(res.stdout.strip().splitlines()[-1])
        cpu = d.get("cpu_baseline") or {}
        thr = cpu.get("threaded") or {}
        row = (f"| {workload} | {' '.join(opts)} | {d['ms_per_step'] * 1e3:.2f} | {d['value']:.4g} | "
               f"{d['elements_per_s']:.4g} | {d['roofline']['frac']:.3f} | "
               f"{cpu.get('value', float('nan')):.4g} | "
               f"{thr.get('value', float('nan')):.4g} ({thr.get('cores', '-')} cores) | "
               f"{d['parity_spot_check']} |")
        print(row, flush=True)
        lines.append(row)
    if out_path:
        with open(out_path, "w") as f:
            f.write("\n".join(lines) + "\n")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("copy")
    c.add_argument("--mib", type=int, default=256)
    c.add_argument("--reps", type=int, default=5)
    m = sub.add_parser("counters")
    m.add_argument("dir")
    m.add_argument("substring")
    s = sub.add_parser("stats")
    s.add_argument("dir")
    t = sub.add_parser("traffic")
    t.add_argument("--workload", required=True)
    t.add_argument("--k", type=int, required=True)
    t.add_argument("--kernel-fetch", required=True)
    t.add_argument("--kernel-write", required=True)
    t.add_argument("--copy-fetch", required=True)
    t.add_argument("--copy-write", required=True)
    t.add_argument("--copy-mib", type=int, default=256)
    t.add_argument("--out", default=None)
    fl = sub.add_parser("floor")
    fl.add_argument("--calls", type=int, default=2000)
    mx = sub.add_parser("matrix")
    mx.add_argument("--out", default=None)
    a = ap.parse_args(argv)

    if a.cmd == "floor":
        run_floor(a.calls)
        return 0
    if a.cmd == "matrix":
        run_matrix(a.out)
        return 0

    if a.cmd == "copy":
        run_copy(a.mib, a.reps)
        return 0
    if a.cmd == "counters":
        for name, (mean, n) in sorted(counter_means(a.dir, a.substring).items()):
            print(f"{name:28s} dispatches={n:6d} mean={mean:16.1f}")
        return 0
    if a.cmd == "stats":
        rows = kernel_stats(a.dir)
        if not rows:
            print("no kernel_stats.csv found", file=sys.stderr)
            return 1
        keys = ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"]
        keys = [k for k in keys if k in rows[0]]
        print(" | ".join(keys))
        for r in rows:
            print(" | ".join(str(r[k]) for k in keys))
        return 0

    # traffic
    known = a.copy_mib * 2**20
    kf = counter_means(a.kernel_fetch, KERNEL_SUBSTRING)["FETCH_SIZE"][0]
    kw = counter_means(a.kernel_write, KERNEL_SUBSTRING)["WRITE_SIZE"][0]
    cf = counter_means(a.copy_fetch, COPY_SUBSTRING)["FETCH_SIZE"][0]
    cw = counter_means(a.copy_write, COPY_SUBSTRING)["WRITE_SIZE"][0]
    fetch_scale, write_scale = known / cf, known / cw
    entry = {
        "hbm_bytes_per_launch": kf * fetch_scale + kw * write_scale,
        "fetch_bytes_per_launch": kf * fetch_scale,
        "write_bytes_per_launch": kw * write_scale,
        "kernel_fetch_kib": kf,
        "kernel_write_kib": kw,
        "copy_fetch_kib": cf,
        "copy_write_kib": cw,
        "copy_bytes_each_way": known,
        "fetch_scale_bytes_per_kib": fetch_scale,
        "write_scale_bytes_per_kib": write_scale,
    }
    key = f"{a.workload}:k={a.k}"
    print(json.dumps({key: entry}, indent=1))
    if a.out:
        table = {}
        if os.path.exists(a.out):
            with open(a.out) as f:
                table = json.load(f)
        table[key] = entry
        with open(a.out, "w") as f:
            json.dump(table, f, indent=1, sort_keys=True)
            f.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
