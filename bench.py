#!/usr/bin/env python3
"""Benchmark PONNI's batched forward pass on one MI355X.

A step is one forward pass of the headline configuration (BASELINE.json
configs[1], "c2": fp32 16->64->64->64->8 ReLU MLP, batch 4,194,304) over a
synthetic input already resident in HBM.  Prints ONE JSON line.

  python bench.py [--steps K] [--warmup W] [--config c2] [--no-others] [--no-cpu]

`value` is samples/s of the whole job (one GPU).  `roofline` prices the
dominant kernel (the only kernel of a step) against MI355X's published peak:
achieved = algorithmic work per sample x batch / mean kernel time, the kernel
time measured with HIP events recorded on the launch stream around each
launch.  `cpu_baseline` times the CPU restatement of the reference (oracle/,
OpenMP over samples, as Kokkos' OpenMP RangePolicy) on a bounded sample on
this host.  Other configurations are reported under "configs".
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "samples/sec/GPU for fused MLP forward; % of HBM or MFMA roofline"
ROTATE_BYTES = 512 << 20  # rotate buffers so the working set exceeds the 256 MB MALL


def pmc_traffic(config_name: str):
    """HBM bytes per launch measured by rocprofv3 PMC runs (profiles/traffic.json)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            entry = json.load(f).get(config_name)
    except (OSError, ValueError):
        return None
    return entry.get("bytes_per_launch") if entry else None


def host_cores() -> int:
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        return int(env)
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


TORCH_DTYPES = {"f32": "float32", "f64": "float64", "f16": "float16", "bf16": "bfloat16"}
ELEMENT_BYTES = {"f32": 4, "f64": 8, "f16": 2, "bf16": 2}


def with_dtype(cfg, dtype, C):
    """The configuration computed in another precision (--dtype): same
    shapes and synthetic inputs, HBM bytes and MFMA peak of that precision."""
    import dataclasses

    if dtype is None or dtype == cfg.dtype:
        return cfg
    scale = ELEMENT_BYTES[dtype] / ELEMENT_BYTES[cfg.dtype]
    peak = cfg.peak
    if cfg.bound == "mfma":
        peak = {"f32": C.FP32_PEAK, "f64": C.FP64_PEAK, "f16": C.FP16_PEAK, "bf16": C.FP16_PEAK}[dtype]
    return dataclasses.replace(cfg, dtype=dtype, peak=peak, bytes_per_sample=int(cfg.bytes_per_sample * scale))


def make_inputs(cfg, torch, P, C):
    tdt = getattr(torch, TORCH_DTYPES[cfg.dtype])
    es = ELEMENT_BYTES[cfg.dtype]
    per_set = (cfg.n_in + cfg.n_out) * cfg.batch * es
    sets = max(1, -(-ROTATE_BYTES // per_set))
    xs, ys = [], []
    for i in range(sets):
        x = torch.empty((cfg.n_in, cfg.batch), dtype=tdt, device="cuda:0")
        kind, a, b = cfg.input_dist
        P.fill_synthetic(x, cfg.seed + 7919 * i, C.INPUT_TAG, kind, a, b)
        xs.append(x)
        ys.append(torch.empty((cfg.n_out, cfg.batch), dtype=tdt, device="cuda:0"))
    return xs, ys


def time_config(cfg, steps, warmup, torch, P, C):
    layers = cfg.layers(False)
    model = P.create_inference_model(*layers, dtype=cfg.dtype)
    xs, ys = make_inputs(cfg, torch, P, C)
    stream = torch.cuda.current_stream()
    B = cfg.batch

    def launch(i):
        x, y = xs[i % len(xs)], ys[i % len(ys)]
        model.forward_raw(x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0), B, stream.cuda_stream)

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    # Whole-job timing: K back-to-back launches.
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        launch(i)
    stop.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    # Per-launch kernel time: events bracket each launch on the launch stream.
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record(stream)
        launch(i)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    per = sorted(a.elapsed_time(b) for a, b in ev)
    mean_ms = sum(per) / len(per)
    work = cfg.flops_per_sample if cfg.bound == "mfma" else cfg.bytes_per_sample
    achieved = work * B / (mean_ms * 1e-3)
    unit = "TFLOP/s" if cfg.bound == "mfma" else "GB/s"
    scale = 1e12 if cfg.bound == "mfma" else 1e9
    return {
        "model": model,
        "layers": layers,
        "samples_per_s": B * steps / (total_ms * 1e-3),
        "ms_per_step": total_ms / steps,
        "kernel_ms_mean": mean_ms,
        "kernel_ms_min": per[0],
        "kernel_ms_median": per[len(per) // 2],
        "roofline": {
            "bound": cfg.bound,
            "achieved": round(achieved / scale, 3),
            "peak": round(cfg.peak / scale, 3),
            "unit": unit,
            "frac": round(achieved / cfg.peak, 4),
            # (PMC traffic is measured for the configurations' own precision only)
            "traffic": pmc_traffic(cfg.name) if cfg.dtype == C.CONFIGS[cfg.name].dtype else None,
        },
        "path": model.path,
    }


def cpu_baseline(cfg, budget_s=10.0):
    """Time the oracle (CPU restatement of the reference) on a bounded sample."""
    import numpy as np

    import oracle
    from ponni_amd import configs as C

    oracle.build()
    layers = cfg.layers(False)
    cores = host_cores()
    mode = {"f16": oracle.MODE_F16_OPERANDS, "bf16": oracle.MODE_BF16_OPERANDS, "f64": oracle.MODE_F64}.get(
        cfg.dtype, oracle.MODE_F32)

    def gen(n):
        kind, a, b = cfg.input_dist
        f = C.uniform if kind == "uniform" else C.normal
        return f(cfg.n_in * n, cfg.seed, C.INPUT_TAG, a, b).reshape(cfg.n_in, n)

    # One pass over the first n columns of the workload's input (n sized from a
    # short probe to take about a tenth of the budget), repeated until the
    # budget is spent.
    n = 16384
    x = gen(n)
    oracle.forward(layers, x, mode, cores)  # warm the thread pool
    t0 = time.perf_counter()
    oracle.forward(layers, x, mode, cores)
    dt = time.perf_counter() - t0
    n = int(min(cfg.batch, 1 << 22, max(n, n * 0.1 * budget_s / max(dt, 1e-6))))
    x = gen(n)
    reps, total = 0, 0.0
    while total < budget_s:
        t0 = time.perf_counter()
        oracle.forward(layers, x, mode, cores)
        total += time.perf_counter() - t0
        reps += 1
    return {
        "value": round(n * reps / total, 1),
        "unit": "samples/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{reps} passes over the first {n} columns of {cfg.name} ({cfg.description}), "
                   f"{total:.1f} s, OpenMP over samples"),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--dtype", choices=sorted(TORCH_DTYPES), default=None,
                    help="run the configuration in another precision (not the headline measurement)")
    ap.add_argument("--no-others", action="store_true", help="skip the other configurations")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a device copy of 256 MiB (reference for PMC byte counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the forward pass shards over the batch with no "
              "collective, and this build runs and reports a single MI355X.", file=sys.stderr)
        return 2

    import torch

    import ponni_amd as P
    from ponni_amd import configs as C

    torch.cuda.init()
    if args.calibrate_copy:
        src = torch.empty(64 << 20, dtype=torch.float32, device="cuda:0")
        P.fill_synthetic(src, 1, 2, "uniform", 0.0, 1.0)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    cfg = with_dtype(C.CONFIGS[args.config], args.dtype, C)
    head = time_config(cfg, args.steps, args.warmup, torch, P, C)
    others = {}
    if not args.no_others:
        for name, c in C.CONFIGS.items():
            if name == cfg.name:
                continue
            r = time_config(c, max(5, args.steps // 2), args.warmup, torch, P, C)
            others[name] = {
                "samples_per_s": round(r["samples_per_s"], 1),
                "kernel_ms_mean": round(r["kernel_ms_mean"], 4),
                "path": r["path"],
                "batch": c.batch,
                "dtype": c.dtype,
                "roofline": r["roofline"],
            }
            del r
            torch.cuda.empty_cache()
    cpu = None if args.no_cpu else cpu_baseline(cfg, args.cpu_seconds)
    line = {
        "metric": METRIC,
        "value": round(head["samples_per_s"], 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": "synthetic",
        "config": {
            "workload": f"{cfg.name}: {cfg.description}",
            "global_batch": cfg.batch,
            "path": head["path"],
            "kernel_ms_mean": round(head["kernel_ms_mean"], 4),
            "kernel_ms_min": round(head["kernel_ms_min"], 4),
            "kernel_ms_median": round(head["kernel_ms_median"], 4),
            "parallelism": "single GPU",
        },
        "roofline": head["roofline"],
        "cpu_baseline": cpu,
        "configs": others,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
