"""Benchmark of the batched fp16 top-k engine on one MI355X.

Default workload: LLM-sampling logits, 128 segments x 128,256 fp16 (N(0, sd 2), 0.1 % of each
row boosted by +8), k = 50.  One step = one call of radix_topk_batch_topk_half over the whole
batch (the inputs already resident in HBM).  The input is replicated over >= 512 MB of
distinct buffers and the timed calls rotate through them, so the 256 MB Infinity Cache cannot
serve the reads; a cache-resident ("warm") timing of a single buffer is reported separately.

Prints ONE JSON line:
  value       = whole-job segments per second over the timed steps;
  roofline    = algorithmic bytes per launch (2 B per input element + 6 B per output rank)
                / the average launch duration over the timed region (HIP events on the launch
                stream around K back-to-back launches), against the 8 TB/s HBM peak;
                traffic = HBM bytes per launch measured with rocprofv3 (profiles/traffic.json);
  cpu_baseline= the reference's host verifier (std::stable_sort per segment, restated in
                oracle/) timed on this host's cores over the whole batch.

Other workloads (--workload uniform_small | ties_special | varlen | huge_segment, and
ref_matrix --seg-num N for the reference's own benchmark matrix) print the same line for
that configuration.  --dtype bf16 runs the bfloat16 entry points on the same workload
rounded to bfloat16 (no CPU baseline: that is the reference's fp16 verifier); --dtype f32 the
float32 entry points on the workload widened to float32 (the same values; 4 bytes per element
in the algorithmic bytes).  --op sample
times the top-k sampling consumer (radix_topk_sample_*: the top-k, then one draw per row
from the softmax of its top-k at --temperature) on fixed-length workloads.  --output times an
output variant of radix_topk_batch_topk_ex (unsorted rows, indices only, or both); its
algorithmic bytes count 4 bytes per output rank when no values are written.

Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--workload NAME] [--k K] [--dtype f16|bf16|f32]
                       [--op topk|sample] [--output sorted|unsorted|indices|unsorted-indices]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_BPS = 8.0e12
METRIC = "segments/s and achieved HBM GB/s, fp16 top-50 over 128×128256 segments"


def log(msg: str) -> None:
    sys.stderr.write(f"[bench] {msg}\n")
    sys.stderr.flush()


def make_input(name: str, seg_num_arg: int | None = None):
    """-> (bits [seg_num, seg_len] or flat for offsets, int32 offsets or None, config dict)."""
    from batch_topk_amd import workloads as wl

    if name == "ref_matrix":
        n = seg_num_arg or 128
        bits = wl.ref_matrix(n)
        return bits, None, dict(workload=f"ref_matrix: {n}x10000 fp16, the reference bench's fill pattern",
                                seg_num=n, seg_len=10000)

    if name == "llm_logits":
        bits = wl.llm_logits()
        return bits, None, dict(workload="llm_logits: 128x128256 fp16 N(0,sd 2), 0.1% of each row +8",
                                seg_num=128, seg_len=128256)
    if name == "uniform_small":
        bits = wl.uniform_small()
        return bits, None, dict(workload="uniform_small: 16x4096 fp16 U(-1,1)", seg_num=16, seg_len=4096)
    if name == "ties_special":
        bits = wl.ties_special()
        return bits, None, dict(workload="ties_special: 256x32000 fp16, 256 distinct values, 1% -inf, 0.1% NaN",
                                seg_num=256, seg_len=32000)
    if name == "huge_segment":
        bits = wl.huge_segment()
        return bits, None, dict(workload="huge_segment: 1x16777216 fp16 N(0,1)", seg_num=1, seg_len=16777216)
    if name == "varlen":
        bits, offsets = wl.varlen()
        return bits, offsets, dict(workload="varlen: 512 segments, lengths U[1,65536], fp16 N(0,1), int32 offsets",
                                   seg_num=512, max_seg_len=65536, elements=int(offsets[-1]))
    raise SystemExit(f"unknown workload {name}")


def load_traffic(workload: str, k: int):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (and scaled by a
    copy kernel of known size), from the committed summary; None if not measured."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        with open(path) as f:
            table = json.load(f)
    except (OSError, ValueError):
        return None
    entry = table.get(f"{workload}:k={k}")
    return None if entry is None else entry.get("hbm_bytes_per_launch")


def offsets_of(workload: str) -> bool:
    return workload == "varlen"


def cpu_baseline(bits: np.ndarray, k: int, threads: int):
    """Reference host verifier over the whole batch, serial (threads=1) and threaded."""
    from oracle import oracle as O  # the checker, timed as the CPU baseline only

    seg_num, seg_len = bits.shape
    t1, _ = O.time_batch_topk_half(bits, k, seg_num, seg_len=seg_len, threads=1, variant=0, reps=3)
    tn, _ = O.time_batch_topk_half(bits, k, seg_num, seg_len=seg_len, threads=threads, variant=0, reps=3)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(value=seg_num / t1, unit="segments/s", cores=1, kind="port",
                sample=f"all {seg_num} segments x {seg_len} (the full batch), std::stable_sort per "
                       f"segment as cpu_reference_topk, median of 3 runs",
                threaded=dict(value=seg_num / tn, unit="segments/s", cores=threads,
                              host_threads_visible=os.cpu_count(),
                              note="one thread per core of the GPU's host-core share (16 per GPU "
                                   "on the measurement boxes); segments split evenly"),
                cpu_model=cpu_model)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="llm_logits")
    ap.add_argument("--k", type=int, default=50)
    ap.add_argument("--seg-num", type=int, default=None, help="segments of the ref_matrix workload")
    ap.add_argument("--rotate-mb", type=int, default=512)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    # The threaded CPU baseline uses the host cores allotted to one GPU (16 on the measurement
    # boxes, whatever os.cpu_count() shows), or fewer if fewer are visible.
    ap.add_argument("--cpu-threads", type=int, default=min(16, os.cpu_count() or 1))
    ap.add_argument("--dtype", choices=("f16", "bf16", "f32"), default="f16")
    ap.add_argument("--op", choices=("topk", "sample"), default="topk")
    ap.add_argument("--temperature", type=float, default=1.0)
    ap.add_argument("--output", choices=("sorted", "unsorted", "indices", "unsorted-indices"),
                    default="sorted", help="output variant of radix_topk_batch_topk_ex (top-k only)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the engine has no "
              f"multi-GPU path", file=sys.stderr)
        return 2

    import torch

    import batch_topk_amd as bt

    bt.load_library()
    dev = torch.device("cuda:0")
    bits, offsets, cfg = make_input(args.workload, args.seg_num)
    k = args.k
    if args.op == "sample" and offsets_of(args.workload):
        raise SystemExit("--op sample runs on fixed-length workloads")
    if args.op == "sample" and args.dtype == "f32":
        raise SystemExit("--op sample takes 16-bit logits")
    flags = {"sorted": 0, "unsorted": bt.UNSORTED, "indices": bt.INDICES_ONLY,
             "unsorted-indices": bt.UNSORTED | bt.INDICES_ONLY}[args.output]
    if flags and args.op == "sample":
        raise SystemExit("--output applies to --op topk")
    ex_format = {"f16": bt.FORMAT_F16, "bf16": bt.FORMAT_BF16, "f32": bt.FORMAT_F32}[args.dtype]
    elem_bytes = 4 if args.dtype == "f32" else 2
    if args.dtype == "bf16":
        # the same workload rounded to bfloat16 (round to nearest even)
        bits = torch.from_numpy(bits.view(np.float16).astype(np.float32)).bfloat16() \
            .view(torch.int16).numpy().view(np.uint16)
        cfg["workload"] += ", rounded to bfloat16"
        fixed, fixed_ws = bt.batch_topk_bf16, bt.batch_topk_bf16_workspace_size
        seg, seg_ws = bt.batch_topk_bf16_segmented, bt.batch_topk_bf16_segmented_workspace_size
    elif args.dtype == "f32":
        # the same workload widened to float32 (exact: the same values, the same top-k)
        bits = bits.view(np.float16).astype(np.float32).view(np.uint32)
        cfg["workload"] += ", widened to float32"
        fixed, fixed_ws = bt.batch_topk_f32, bt.batch_topk_f32_workspace_size
        seg, seg_ws = bt.batch_topk_f32_segmented, bt.batch_topk_f32_segmented_workspace_size
    else:
        fixed, fixed_ws = bt.batch_topk_half, bt.batch_topk_half_workspace_size
        seg, seg_ws = bt.batch_topk_half_segmented, bt.batch_topk_half_segmented_workspace_size
    if offsets is None:
        seg_num, seg_len = bits.shape
        n_elements = seg_num * seg_len
        ws_bytes = fixed_ws(seg_num, seg_len, k)
    else:
        seg_num, seg_len = offsets.size - 1, int(np.max(np.diff(offsets)))
        n_elements = int(offsets[-1])
        ws_bytes = seg_ws(seg_num, cfg["max_seg_len"], k)
        d_off = torch.from_numpy(offsets.astype(np.int32)).to(dev)
    if ws_bytes == 0:
        raise SystemExit(f"shape not supported: {cfg} k={k}")
    in_bytes = bits.nbytes
    copies = max(1, -(-args.rotate_mb * 2**20 // in_bytes))
    log(f"workload {cfg['workload']} k={k}, {copies} input copies ({copies * in_bytes / 2**20:.0f} MB)")
    src = torch.from_numpy(bits.view(np.int32 if elem_bytes == 4 else np.int16)).to(dev)
    inputs = [src] + [src.clone() for _ in range(copies - 1)]
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    vals = torch.empty((seg_num, k), dtype=torch.int32 if elem_bytes == 4 else torch.int16, device=dev)
    idx = torch.empty((seg_num, k), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    if args.op == "sample":
        sample_fn = bt.sample_half if args.dtype == "f16" else bt.sample_bf16
        uniforms = torch.rand(seg_num, dtype=torch.float32, device=dev, generator=torch.Generator(dev).manual_seed(0))
        samples = torch.empty(seg_num, dtype=torch.int32, device=dev)

    def call(i: int) -> None:
        if args.op == "sample":
            rc = sample_fn(inputs[i % copies].data_ptr(), seg_num, seg_len, k, args.temperature,
                           uniforms.data_ptr(), vals.data_ptr(), idx.data_ptr(), 0, samples.data_ptr(),
                           ws.data_ptr(), ws_bytes, sh)
        elif flags:
            rc = bt.batch_topk_ex(inputs[i % copies].data_ptr(), ex_format,
                                  0 if offsets is None else d_off.data_ptr(), seg_num,
                                  seg_len if offsets is None else cfg["max_seg_len"], k, flags,
                                  0 if flags & bt.INDICES_ONLY else vals.data_ptr(), idx.data_ptr(),
                                  ws.data_ptr(), ws_bytes, sh)
        elif offsets is None:
            rc = fixed(inputs[i % copies].data_ptr(), seg_num, seg_len, k, vals.data_ptr(),
                       idx.data_ptr(), ws.data_ptr(), ws_bytes, sh)
        else:
            rc = seg(inputs[i % copies].data_ptr(), d_off.data_ptr(), seg_num, cfg["max_seg_len"], k,
                     vals.data_ptr(), idx.data_ptr(), ws.data_ptr(), ws_bytes, sh)
        if rc != 0:
            raise RuntimeError(f"top-k call returned {rc}")

    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()

    # Parity spot check of the measured configuration (first segments, oracle as checker).
    from oracle import oracle as O

    call(0)
    torch.cuda.synchronize()
    if offsets is None:
        ev, ei = O.batch_topk_half(bits[:8], k, seg_len=seg_len, fmt=args.dtype)
    else:
        ev, ei = O.batch_topk_half(bits[:int(offsets[8])], k, offsets=offsets[:9].astype(np.int64),
                                   fmt=args.dtype)
    gi = idx.cpu().numpy()[:8]
    gv = vals.cpu().numpy().view(np.uint32 if elem_bytes == 4 else np.uint16)[:8]
    if flags & bt.UNSORTED:
        # the same (index, value) set per row, in any order (pads: index -1 sorts first)
        go, eo = np.argsort(gi, axis=1, kind="stable"), np.argsort(ei, axis=1, kind="stable")
        gi, ei = np.take_along_axis(gi, go, 1), np.take_along_axis(ei, eo, 1)
        gv, ev = np.take_along_axis(gv, go, 1), np.take_along_axis(ev, eo, 1)
    parity_ok = bool(np.array_equal(gi, ei) and (bool(flags & bt.INDICES_ONLY) or np.array_equal(gv, ev)))
    log(f"parity spot check (8 segments vs oracle): {'ok' if parity_ok else 'MISMATCH'}")

    # Timed region: K back-to-back steps, events on the launch stream.
    steps = args.steps
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(steps):
        call(i)
    stop.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    ms_per_step = total_ms / steps

    # Per-launch durations (events bracketing each launch), cold (rotating) and warm.
    def per_launch(n: int, rotate: bool):
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(2 * n)]
        torch.cuda.synchronize()
        for i in range(n):
            evs[2 * i].record(stream)
            call(i if rotate else 0)
            evs[2 * i + 1].record(stream)
        torch.cuda.synchronize()
        return np.array([evs[2 * i].elapsed_time(evs[2 * i + 1]) for i in range(n)]) * 1e3  # us

    cold_us = per_launch(max(100, min(steps, 400)), True)  # median of >= 100 calls
    warm_us = per_launch(100, False)
    kern_us = float(np.median(cold_us))

    # Algorithmic bytes: every input element read once (2 B, 4 B for fp32), every output rank
    # written once (value of the element's size + 4 B index), plus the offsets array when given.
    out_bytes = 4 + (0 if flags & bt.INDICES_ONLY else elem_bytes)
    alg_bytes = elem_bytes * n_elements + out_bytes * seg_num * k + (0 if offsets is None else 4 * (seg_num + 1))
    if args.op == "sample":
        alg_bytes += 8 * seg_num  # one uniform in, one sampled index out per row
    # The kernel's average launch duration over the timed region (back-to-back launches,
    # events on the launch stream).
    step_us = ms_per_step * 1e3
    achieved = alg_bytes / (step_us * 1e-6)
    value = seg_num * steps / (total_ms * 1e-3)
    dname = {"f16": "fp16", "bf16": "bf16", "f32": "fp32"}[args.dtype]
    metric = METRIC if (args.workload == "llm_logits" and k == 50 and args.dtype == "f16" and args.op == "topk"
                        and not flags) else \
        f"segments/s and achieved HBM GB/s, {dname} top-{k}{' sampling' if args.op == 'sample' else ''} " \
        f"over {cfg['workload'].split(':')[0]}{'' if not flags else f' ({args.output} output)'}"
    result = {
        "metric": metric,
        "value": value,
        "unit": "segments/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"f16": "fp16", "bf16": "bf16", "f32": "fp32"}[args.dtype],
        "data": "synthetic",
        "config": dict(cfg, k=k, input_copies=copies, parallelism="single GPU",
                       **({"output": args.output} if flags else {}),
                       **({"op": "top-k sampling", "temperature": args.temperature} if args.op == "sample" else {})),
        "roofline": {
            "bound": "hbm",
            "achieved": achieved / 1e9,
            "peak": HBM_PEAK_BPS / 1e9,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_BPS,
            "traffic": load_traffic(args.workload if args.dtype == "f16" else f"{args.workload}:{args.dtype}", k)
            if args.op == "topk" and not flags else None,
        },
        "elements_per_s": n_elements * steps / (total_ms * 1e-3),
        "hbm_gbps_whole_job": alg_bytes * steps / (total_ms * 1e-3) / 1e9,
        "kernel_us_isolated_median": kern_us,
        "kernel_us_p10_p90": [float(np.percentile(cold_us, 10)), float(np.percentile(cold_us, 90))],
        "warm_kernel_us_isolated_median": float(np.median(warm_us)),
        "alg_bytes_per_launch": alg_bytes,
        "parity_spot_check": parity_ok,
    }
    if args.workload == "ref_matrix":
        from batch_topk_amd.workloads import REF_MATRIX_TARGET_US

        target = REF_MATRIX_TARGET_US.get((seg_num, seg_len, k))
        result["reference_target_us_rtx4080"] = target
        result["target_over_measured"] = None if target is None else target / (ms_per_step * 1e3)
    if not args.no_cpu_baseline and offsets is None and args.dtype == "f16" and args.op == "topk" and not flags:
        log("timing the CPU baseline (reference host verifier)...")
        t0 = time.time()
        result["cpu_baseline"] = cpu_baseline(bits, k, args.cpu_threads)
        log(f"cpu baseline done in {time.time() - t0:.1f} s")
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result))
    sys.stdout.flush()
    return 0 if parity_ok else 1


if __name__ == "__main__":
    sys.exit(main())
