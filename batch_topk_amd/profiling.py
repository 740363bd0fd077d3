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
      fp16 batch, rotating over 17 input copies (557 MB), for several workgroup shapes; the
      per-wave arrival order of one workgroup's loads; the asymptotic streaming rate.

  python -m batch_topk_amd.profiling matrix [--out FILE]
      bench.py over every workload (fp16; bf16 and the sampling consumer on the LLM logits;
      fp32 on every workload; the unsorted and indices-only outputs), as a markdown table.

  python -m batch_topk_amd.profiling phases [--workload W | --shape SEGxLEN] [--k K] [--b2b N]
        [--per-wave]
      Step timeline of the top-k kernel on an fp16 workload, from the phase-traced build of
      the engine (libbatch_topk_amd_trace.so): per-workgroup stamps of the last of N
      back-to-back calls, on the GPU's constant 100 MHz clock from the first workgroup's
      start, and per-wave stamps on the shader clock from the wave's workgroup start (with
      --per-wave also the median of each wave step by wave index).  The stamps cost time
      themselves (the traced build runs about 1 us slower per call).
"""

from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import os
import sys
import warnings

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
    # Per-wave arrival: in what order one CU serves the loads of a 1024-thread workgroup.
    lib.read_floor_arrival_run.restype = i32
    lib.read_floor_arrival_run.argtypes = [vp, i32, i32, i32, i32, vp, vp, vp]
    stamps = torch.zeros(rows * 16 * 3, dtype=torch.int64, device="cuda:0")
    aout = torch.empty(rows * 16, dtype=torch.int32, device="cuda:0")
    print("per-wave arrival, 1 workgroup of 1024 threads x 16 vectors per row (median over the "
          f"{rows} workgroups of the last of 200 back-to-back launches; ns from the workgroup's first wave start)")
    for barrier_first in (0, 1):
        rc = lib.read_floor_arrival_run(ptrs, 200, rows, row_len, barrier_first, aout.data_ptr(),
                                        stamps.data_ptr(), stream.cuda_stream)
        if rc != 0:
            raise RuntimeError(f"read_floor_arrival_run returned {rc}")
        torch.cuda.synchronize()
        S = stamps.view(rows, 16, 3).cpu().numpy().astype(np.int64)
        # the shader clock runs at about 2.4 GHz on this part
        rel = (S - S[:, :, 0].min(axis=1)[:, None, None]) / 2.4
        print(f"{'barrier before the loads' if barrier_first else 'no barrier'}: wave | "
              + " ".join(f"{w:5d}" for w in range(16)))
        for col, name in ((0, "start"), (1, "loads issued"), (2, "data in")):
            print(f"  {name:12s} | " + " ".join(f"{x:5.0f}" for x in np.median(rel[:, :, col], axis=0)))
    # Asymptotic streaming rate: the same loads over 512 MiB per launch (2048 rows of 131,072
    # fp16, two buffers alternating), where the launch cost and the ramp are a few percent.
    big_rows, big_len = 2048, 131072
    big = [torch.empty(big_rows * big_len, dtype=torch.int16, device="cuda:0") for _ in range(2)]
    for t in big:
        t.fill_(1)
    big_calls = 40
    bptrs = (ctypes.c_void_p * big_calls)(*[big[i % 2].data_ptr() for i in range(big_calls)])
    bout = torch.empty(big_rows * 4 * 16, dtype=torch.int32, device="cuda:0")
    big_bytes = 2 * big_rows * big_len
    print(f"streaming read of {big_rows} x {big_len} fp16 ({big_bytes} bytes) per launch, "
          f"{big_calls} back-to-back launches over 2 buffers")
    print("workgroups per row | threads x vectors | us per launch | GB/s | fraction of 8 TB/s")
    for block, vpt, w in ((1024, 16, 1), (512, 16, 2), (256, 16, 4)):
        def go_big():
            rc = lib.read_floor_run(bptrs, big_calls, big_rows, big_len, block, vpt, w, bout.data_ptr(),
                                    stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"read_floor_run returned {rc}")
        go_big()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        go_big()
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / big_calls
        print(f"{w} | {block} x {vpt} | {us:.2f} | {big_bytes / us / 1e3:.0f} | "
              f"{big_bytes / us / 1e3 / 8000:.3f}")


PHASES = ((12, "loads issued"), (1, "thread best"), (2, "first histogram round"),
          (8, "first meeting / list published"), (9, "cooperative threshold"), (4, "threshold"),
          (5, "filter"), (6, "refinement done"), (10, "list stored / lists merged"),
          (3, "cooperative lengths read"), (7, "cooperative lists gathered"), (11, "end"))
WAVE_PHASES = ((1, "thread best"), (0, "threshold read"), (2, "filter start"), (3, "vectors staged"),
               (4, "flushed"), (5, "after filter barrier"), (6, "ranking start"), (7, "ranking end"))


def run_phases(workload: str, k: int, b2b: int, shape: str | None = None, per_wave: bool = False) -> None:
    import ctypes

    import numpy as np
    import torch

    from batch_topk_amd import build, workloads

    lib = ctypes.CDLL(build.TRACE_LIB_PATH)
    vp, i32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    lib.radix_topk_trace_fetch.argtypes = [vp, vp, vp]
    lib.radix_topk_trace_fetch.restype = i32
    lib.radix_topk_trace_clear.argtypes = []
    lib.radix_topk_trace_clear.restype = i32
    if shape:  # SEGxLEN of N(0, 1) fp16, seed 0
        seg_num_s, seg_len_s = (int(v) for v in shape.lower().split("x"))
        rng = np.random.default_rng(0)
        out = rng.standard_normal((seg_num_s, seg_len_s), dtype=np.float32).astype(np.float16).view(np.uint16)
        workload = f"N(0,1) {seg_num_s}x{seg_len_s}"
    else:
        out = getattr(workloads, workload)()
    if isinstance(out, tuple):  # varlen: (bits, offsets)
        bits, offsets = out
        seg_num, max_len = offsets.size - 1, int(np.diff(offsets).max())
    else:
        bits, offsets = out, None
        seg_num, max_len = bits.shape
    dev = "cuda:0"
    src = torch.from_numpy(np.ascontiguousarray(bits).reshape(-1).view(np.int16)).to(dev)
    copies = [src] + [src.clone() for _ in range(max(1, -(-512 * 2**20 // (2 * src.numel()))) - 1)]
    vals = torch.empty((seg_num, k), dtype=torch.int16, device=dev)
    idx = torch.empty((seg_num, k), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    if offsets is None:
        lib.radix_topk_batch_topk_half_workspace_size.restype = sz
        lib.radix_topk_batch_topk_half_workspace_size.argtypes = [i32, i32, i32]
        lib.radix_topk_batch_topk_half.argtypes = [vp, i32, i32, i32, vp, vp, vp, sz, vp]
        wsb = lib.radix_topk_batch_topk_half_workspace_size(seg_num, max_len, k)
    else:
        lib.radix_topk_batch_topk_half_segmented_workspace_size.restype = sz
        lib.radix_topk_batch_topk_half_segmented_workspace_size.argtypes = [i32, i32, i32]
        lib.radix_topk_batch_topk_half_segmented.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp, sz, vp]
        wsb = lib.radix_topk_batch_topk_half_segmented_workspace_size(seg_num, max_len, k)
        d_off = torch.from_numpy(offsets.astype(np.int32)).to(dev)
    ws = torch.empty(max(1, wsb), dtype=torch.uint8, device=dev)

    def call(i):
        x = copies[i % len(copies)].data_ptr()
        if offsets is None:
            rc = lib.radix_topk_batch_topk_half(x, seg_num, max_len, k, vals.data_ptr(), idx.data_ptr(),
                                                ws.data_ptr(), wsb, stream)
        else:
            rc = lib.radix_topk_batch_topk_half_segmented(x, d_off.data_ptr(), seg_num, max_len, k,
                                                          vals.data_ptr(), idx.data_ptr(), ws.data_ptr(), wsb, stream)
        if rc != 0:
            raise RuntimeError(f"top-k call returned {rc}")

    for i in range(30):
        call(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(200):
        call(i)
    b.record()
    torch.cuda.synchronize()
    print(f"{workload} k={k}, phase-traced build: {a.elapsed_time(b) * 1e3 / 200:.2f} us per call back-to-back")
    nwg, nslot = 2048, 16
    clock = np.zeros(nwg * nslot, np.uint64)
    real = np.zeros(nwg * nslot, np.uint64)
    wave = np.zeros(nwg * nslot * 16, np.uint64)
    if lib.radix_topk_trace_clear() != 0:
        raise RuntimeError("trace clear failed")
    for i in range(b2b):
        call(i)
    torch.cuda.synchronize()
    if lib.radix_topk_trace_fetch(clock.ctypes.data, real.ctypes.data, wave.ctypes.data) != 0:
        raise RuntimeError("trace fetch failed")
    C = clock.reshape(nwg, nslot).astype(np.int64)
    R = real.reshape(nwg, nslot).astype(np.int64)
    W = wave.reshape(nwg, nslot, 16).astype(np.int64)
    g = np.nonzero(R[:, 0])[0]
    C, R, W = C[g], R[g], W[g]
    r0 = R[:, 0].min()
    print(f"last of {b2b} back-to-back calls: {len(g)} workgroups stamped")
    print("workgroup step (ns from the first workgroup's start) | stamped | min | median | p90 | max")

    def row(name, d):
        print(f"{name} | {d.size} | {d.min():.0f} | {np.median(d):.0f} | {np.percentile(d, 90):.0f} | {d.max():.0f}")

    row("start", (R[:, 0] - r0) * 10.0)
    stamped = [(np.median(R[R[:, j] > 0, j]), j, name) for j, name in PHASES if np.any(R[:, j] > 0)]
    for _, j, name in sorted(stamped):  # in the order the steps ran
        m = R[:, j] > 0
        row(name, (R[m, j] - r0) * 10.0)
    end = np.where(R[:, 11] > 0, R[:, 11], R.max(axis=1))
    ok = (C[:, 11] > C[:, 0]) & (end > R[:, 0])
    if ok.any():
        ticks_per_ns = np.median((C[ok, 11] - C[ok, 0]) / ((R[ok, 11] - R[ok, 0]) * 10.0))
        print(f"wave step (ns from its workgroup's start; shader clock {ticks_per_ns * 1e3:.0f} MHz) | stamped | min | median | p90 | max")
        for j, name in WAVE_PHASES:
            m = W[:, :, j] > 0
            if m.any():
                row(name, ((W[:, :, j] - C[:, 0:1]) / ticks_per_ns)[m])
        if per_wave:
            print("wave step by wave index (median ns from its workgroup's start over the workgroups; waves 0..15)")
            for j, name in WAVE_PHASES:
                m = W[:, :, j] > 0
                if m.any():
                    t = np.where(m, (W[:, :, j] - C[:, 0:1]) / ticks_per_ns, np.nan)
                    with np.errstate(all="ignore"), warnings.catch_warnings():
                        warnings.simplefilter("ignore", RuntimeWarning)  # waves that never stamp j
                        med = np.nanmedian(t, axis=0)
                    print(f"{name:22s} " + " ".join("    -" if np.isnan(x) else f"{x:5.0f}" for x in med))
    cand = C[:, 14][C[:, 14] > 0]
    if cand.size:
        print(f"candidates per workgroup: min {cand.min()} median {np.median(cand):.0f} max {cand.max()}")


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
    ph = sub.add_parser("phases")
    ph.add_argument("--workload", default="llm_logits")
    ph.add_argument("--k", type=int, default=50)
    ph.add_argument("--b2b", type=int, default=20)
    ph.add_argument("--shape", default=None, help="SEGxLEN of N(0,1) fp16 instead of a workload")
    ph.add_argument("--per-wave", action="store_true", help="also the median of every wave step by wave index")
    a = ap.parse_args(argv)

    if a.cmd == "phases":
        run_phases(a.workload, a.k, a.b2b, a.shape, a.per_wave)
        return 0

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
