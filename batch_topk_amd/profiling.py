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
    a = ap.parse_args(argv)

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
