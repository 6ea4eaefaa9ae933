#!/usr/bin/env python3
"""Benchmark PONNI's batched forward pass on one MI355X.

A step is one forward pass of the headline configuration over a synthetic
input already resident in HBM.  The headline is "c4", the largest
configuration of BASELINE.json (fp16 MLP 64->256->256->256->64 with tanh,
fp16 operands and fp32 accumulation, batch 8,388,608); every other
configuration is measured the same way and reported under "configs".
Prints ONE JSON line.

  python bench.py [--steps K] [--warmup W] [--config c4] [--no-others] [--no-cpu]
  python bench.py --trace-summary run_kernel_trace.csv --skip W   (rocprofv3 output)

Timing.  W untimed launches, then K timed launches back to back on one stream.
Each timed launch goes through ponni_forward_timed, whose dispatch stamps two
HIP events with the kernel's own start and end; two more events bracket the K
launches.  `ms_per_step` = bracket / K and `value` = batch / ms_per_step.
`roofline.achieved` = algorithmic work per sample x batch / the kernel's mean
duration over the same K launches (`frac`); `frac_per_step` prices the same
work on ms_per_step.  `roofline.traffic` = HBM bytes per launch from the
committed rocprofv3 PMC runs (profiles/traffic.json).  `cpu_baseline` times the
CPU restatement of the reference (oracle/, OpenMP over samples as Kokkos'
OpenMP RangePolicy) on a bounded sample of each configuration on this host.
`measured_peaks` reports a device copy's and register-only MFMA loops' rates
measured on the same GPU, beside the published peaks `frac` is priced on.
"""
from __future__ import annotations

import argparse
import csv
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "samples/sec/GPU for fused MLP forward; % of HBM or MFMA roofline"
HEADLINE = "c4"
ROTATE_BYTES = 512 << 20  # rotate buffers so the working set exceeds the 256 MB MALL
C1_LARGE_BATCH = 64 << 20  # supplementary c1 entry: the same net over 67,108,864 samples


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


class HipEvents:
    """HIP events through the runtime this process already loaded (torch's)."""

    def __init__(self):
        path = None
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64.so" in line:
                    path = line.split()[-1]
                    break
        if path is None:
            raise RuntimeError("the HIP runtime is not loaded")
        L = ctypes.CDLL(path)
        vp = ctypes.c_void_p
        L.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        L.hipEventDestroy.argtypes = [vp]
        L.hipEventRecord.argtypes = [vp, vp]
        L.hipEventSynchronize.argtypes = [vp]
        L.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        self.L = L

    def create(self) -> int:
        ev = ctypes.c_void_p()
        self._ok(self.L.hipEventCreate(ctypes.byref(ev)), "hipEventCreate")
        return ev.value

    def destroy(self, ev: int) -> None:
        self.L.hipEventDestroy(ev)

    def record(self, ev: int, stream: int) -> None:
        self._ok(self.L.hipEventRecord(ev, stream), "hipEventRecord")

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = ctypes.c_float()
        self._ok(self.L.hipEventElapsedTime(ctypes.byref(ms), a, b), "hipEventElapsedTime")
        return float(ms.value)

    @staticmethod
    def _ok(rc: int, what: str) -> None:
        if rc != 0:
            raise RuntimeError(f"{what} failed with HIP error {rc}")


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


SMALL_LAUNCH_BYTES = 64 << 20  # HBM-bound launches up to this size are priced on the 12 MB copy


def frac_of_measured(pk, roofline, dtype, launch_bytes=None):
    """A kernel's achieved rate over the measured rate of the unit that bounds it
    (HBM: the faster of the 1 GiB copy and the read-only pass, or for a launch
    of at most SMALL_LAUNCH_BYTES the c1-shaped 12 MB copy, whose time is
    mostly launch and DRAM latency; None where no matching rate is measured,
    e.g. fp64 MFMA)."""
    small = launch_bytes is not None and launch_bytes <= SMALL_LAUNCH_BYTES
    bound = {"hbm": pk.hbm_copy_12mb_gbps if small else max(pk.hbm_copy_gbps, pk.hbm_read_gbps),
             "mfma": {"f16": pk.mfma_f16_tflops, "bf16": pk.mfma_f16_tflops,
                      "f32": pk.mfma_f32_tflops}.get(dtype)}[roofline["bound"]]
    return round(roofline["achieved"] / bound, 4) if bound else None


def measured_peaks(roofline, cfg, others):
    """Copy and MFMA rates measured on this device (ponni_measure_peaks), and the
    headline kernel's rate as a fraction of the one that bounds it; each other
    configuration's roofline gets the same `frac_of_measured`.  Reported beside
    the published peaks; `roofline.frac` stays priced on the published one."""
    from ponni_amd import _abi as A

    pk = A.Peaks()
    A.check(A.lib().ponni_measure_peaks(ctypes.byref(pk), None))
    for o in others.values():
        o["roofline"]["frac_of_measured"] = frac_of_measured(pk, o["roofline"], o["dtype"], o.get("launch_bytes"))
    out = {
        "hbm_copy_GBps": round(pk.hbm_copy_gbps, 1),
        "hbm_read_GBps": round(pk.hbm_read_gbps, 1),
        "hbm_copy_12MB_GBps": round(pk.hbm_copy_12mb_gbps, 1),
        "copy_12MB_us": round(pk.copy_12mb_us, 3),
        "mfma_f16_TFLOPs": round(pk.mfma_f16_tflops, 1),
        "mfma_f32_TFLOPs": round(pk.mfma_f32_tflops, 1),
        "method": ("1 GiB device copy, the faster of two launch shapes (bytes read + written); "
                   "read-only pass over 1 GiB; HBM-bound kernels priced on the faster of the two; "
                   "a copy of c1's traffic at c1's launch shape (1,000,000 columns, 8 MB read from two rows, "
                   "4 MB written, 16-byte lanes, 48 sets in rotation, mean of the dispatches' own durations), "
                   "which prices HBM-bound launches of at most 64 MiB; register-only loops of "
                   "v_mfma_f32_16x16x32_f16 and v_mfma_f32_16x16x4f32, one 512-thread workgroup "
                   "per CU; medians of 3-5 samples of 2-4 back-to-back launches"),
    }
    out["frac_of_measured"] = frac_of_measured(pk, roofline, cfg.dtype, cfg.bytes_per_sample * cfg.batch)
    return out


def time_config(cfg, steps, warmup, torch, P, C, ev):
    layers = cfg.layers(False)
    model = P.create_inference_model(*layers, dtype=cfg.dtype)
    xs, ys = make_inputs(cfg, torch, P, C)
    stream = torch.cuda.current_stream().cuda_stream
    B = cfg.batch

    def args(i):
        x, y = xs[i % len(xs)], ys[i % len(ys)]
        return x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0), B, stream

    for i in range(warmup):
        model.forward_raw(*args(i))
    torch.cuda.synchronize()
    starts = [ev.create() for _ in range(steps)]
    stops = [ev.create() for _ in range(steps)]
    t0, t1 = ev.create(), ev.create()
    # The rotation continues past the warm-up's buffer sets, so no timed
    # launch finds its input still in the MALL from a recent launch; the
    # launches' arguments are formed before the timed region.
    launches = [(*args(warmup + i), starts[i], stops[i]) for i in range(steps)]
    try:
        ev.record(t0, stream)
        for a in launches:
            model.forward_raw_timed(*a)
        ev.record(t1, stream)
        torch.cuda.synchronize()
        total_ms = ev.elapsed_ms(t0, t1)
        per = [ev.elapsed_ms(a, b) for a, b in zip(starts, stops)]
    finally:
        for e in starts + stops + [t0, t1]:
            ev.destroy(e)
    ms_per_step = total_ms / steps
    kernel_ms = sum(per) / len(per)
    # The same number of launches over the same buffer rotation, issued by the
    # library's own host code (ponni_forward_steps): the per-step time of the C
    # ABI path, without the Python call in between.
    from ponni_amd import _abi as A

    xp = (ctypes.c_void_p * len(xs))(*[x.data_ptr() for x in xs])
    yp = (ctypes.c_void_p * len(ys))(*[y.data_ptr() for y in ys])
    cabi = ctypes.c_double()
    A.check(A.lib().ponni_forward_steps(model._plan, xp, xs[0].stride(0), yp, ys[0].stride(0), B, len(xs), steps,
                                        stream, ctypes.byref(cabi)))
    work = cfg.flops_per_sample if cfg.bound == "mfma" else cfg.bytes_per_sample
    registered = {**C.CONFIGS, **C.SUPPLEMENTARY}.get(cfg.name)
    unit = "TFLOP/s" if cfg.bound == "mfma" else "GB/s"
    scale = 1e12 if cfg.bound == "mfma" else 1e9
    achieved = work * B / (kernel_ms * 1e-3)
    per_sorted = sorted(per)
    return {
        "layers": layers,
        "samples_per_s": B / (ms_per_step * 1e-3),
        "ms_per_step": ms_per_step,
        "ms_per_step_c_abi": cabi.value,
        "kernel_ms_mean": kernel_ms,
        "kernel_ms_min": per_sorted[0],
        "kernel_ms_median": statistics.median(per_sorted),
        "roofline": {
            "bound": cfg.bound,
            "achieved": round(achieved / scale, 3),
            "peak": round(cfg.peak / scale, 3),
            "unit": unit,
            "frac": round(achieved / cfg.peak, 4),
            "frac_per_step": round(work * B / (ms_per_step * 1e-3) / cfg.peak, 4),
            # (PMC traffic is measured for the configurations' own precision and batch only)
            "traffic": (pmc_traffic(cfg.name) if registered is not None and cfg.dtype == registered.dtype
                        and cfg.batch == registered.batch else None),
        },
        "path": model.path,
    }


ORACLE_MODE_NAMES = {"f32": "fp32", "f64": "fp64", "f16": "fp16 operands, fp32 accumulation",
                     "bf16": "bf16 operands, fp32 accumulation"}


def cpu_baseline(cfg, budget_s):
    """Time the oracle (CPU restatement of the reference) on a bounded sample."""
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

    # One pass over n columns drawn from the workload's input distribution (n
    # sized from a short probe to take about a tenth of the budget), repeated
    # until the budget is spent.
    n = 4096
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
        "sample": (f"{reps} passes over {n} columns of {cfg.name} ({cfg.description}; same input distribution), "
                   f"{total:.1f} s, {ORACLE_MODE_NAMES[cfg.dtype]}, OpenMP over samples on {cores} threads"),
    }


def summarize_trace(path: str, skip: int) -> int:
    """Per-kernel statistics of a rocprofv3 kernel trace (CSV), one row per
    kernel and grid size (one configuration), leaving out the first `skip`
    dispatches of each (the bench's untimed warm-up)."""
    rows = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            d = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            key = (r["Kernel_Name"], int(r["Grid_Size_X"]))
            rows.setdefault(key, []).append((int(r["Start_Timestamp"]), d))
    print(f"| Kernel | Grid (work-items) | Dispatches (after skipping {skip}) | Average ns | Median ns | Min ns | "
          "Max ns |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for (name, grid), v in sorted(rows.items(), key=lambda kv: -sum(d for _, d in kv[1])):
        v.sort()
        d = [x for _, x in v[skip:]] or [x for _, x in v]
        print(f"| `{name[:90]}` | {grid:,} | {len(d)} | {sum(d) / len(d):,.0f} | {statistics.median(d):,.0f} | "
              f"{min(d):,} | {max(d):,} |")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default=HEADLINE)
    ap.add_argument("--batch", type=int, default=None, help="override the configuration's batch (not a headline)")
    ap.add_argument("--dtype", choices=sorted(TORCH_DTYPES), default=None,
                    help="run the configuration in another precision (not the headline measurement)")
    ap.add_argument("--no-others", action="store_true", help="skip the other configurations")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU budget of the headline configuration")
    ap.add_argument("--cpu-seconds-others", type=float, default=6.0, help="CPU budget of each other configuration")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured copy and MFMA peaks")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a device copy of 256 MiB (reference for PMC byte counters)")
    ap.add_argument("--trace-summary", metavar="CSV", help="summarize a rocprofv3 kernel trace and exit")
    ap.add_argument("--skip", type=int, default=3, help="with --trace-summary: dispatches to drop per kernel")
    args = ap.parse_args()
    if args.trace_summary:
        return summarize_trace(args.trace_summary, args.skip)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the forward pass shards over the batch with no "
              "collective, and this build runs and reports a single MI355X.", file=sys.stderr)
        return 2

    import dataclasses

    import torch

    import ponni_amd as P
    from ponni_amd import configs as C

    torch.cuda.init()
    ev = HipEvents()
    if args.calibrate_copy:
        src = torch.empty(64 << 20, dtype=torch.float32, device="cuda:0")
        P.fill_synthetic(src, 1, 2, "uniform", 0.0, 1.0)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    cfg = with_dtype({**C.CONFIGS, **C.SUPPLEMENTARY}[args.config], args.dtype, C)
    if args.batch:
        cfg = dataclasses.replace(cfg, batch=args.batch)
    head = time_config(cfg, args.steps, args.warmup, torch, P, C, ev)
    torch.cuda.empty_cache()
    others = {}
    if not args.no_others:
        runs = [(name, c) for name, c in C.CONFIGS.items() if name != cfg.name]
        runs.append(("c1_large", dataclasses.replace(
            C.CONFIGS["c1"], batch=C1_LARGE_BATCH,
            description=C.CONFIGS["c1"].description + ", supplementary batch of 67,108,864 (not a BASELINE config)")))
        runs += list(C.SUPPLEMENTARY.items())
        for name, c in runs:
            r = time_config(c, max(10, args.steps // 2), args.warmup, torch, P, C, ev)
            others[name] = {
                "workload": c.description,
                "batch": c.batch,
                "dtype": c.dtype,
                "path": r["path"],
                "samples_per_s": round(r["samples_per_s"], 1),
                "ms_per_step": round(r["ms_per_step"], 5),
                "ms_per_step_c_abi": round(r["ms_per_step_c_abi"], 5),
                "launch_bytes": c.bytes_per_sample * c.batch,
                "kernel_ms_mean": round(r["kernel_ms_mean"], 5),
                "kernel_ms_min": round(r["kernel_ms_min"], 5),
                "kernel_ms_median": round(r["kernel_ms_median"], 5),
                "roofline": r["roofline"],
            }
            del r
            torch.cuda.empty_cache()
    peaks = None if args.no_peaks else measured_peaks(head["roofline"], cfg, others)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg, args.cpu_seconds)
        for name in others:
            if name in C.CONFIGS:
                others[name]["cpu_baseline"] = cpu_baseline(C.CONFIGS[name], args.cpu_seconds_others)
    line = {
        "metric": METRIC,
        "value": round(head["samples_per_s"], 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg.dtype,
        "data": "synthetic",
        "config": {
            "workload": f"{cfg.name}: {cfg.description}",
            "global_batch": cfg.batch,
            "path": head["path"],
            "ms_per_step_c_abi": round(head["ms_per_step_c_abi"], 5),
            "kernel_ms_mean": round(head["kernel_ms_mean"], 5),
            "kernel_ms_min": round(head["kernel_ms_min"], 5),
            "kernel_ms_median": round(head["kernel_ms_median"], 5),
            "parallelism": "single GPU",
        },
        "roofline": head["roofline"],
        "measured_peaks": peaks,
        "cpu_baseline": cpu,
        "configs": others,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
