"""bench.py's contract: one JSON line with the driver's keys plus `roofline`,
`measured_peaks` and `cpu_baseline`; more than one GPU refused before any
device work; the rocprofv3 trace summary leaves out each kernel's warm-up
dispatches.  The GPU test runs bench.py as a child process on c2 with two
timed steps."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""


def test_trace_summary_skips_warmup_dispatches(tmp_path):
    rows = ["Kernel_Name,Grid_Size_X,Start_Timestamp,End_Timestamp"]
    for i in range(5):  # 2 warm-up dispatches (100 ns), 3 timed (200, 300, 400 ns)
        d = 100 if i < 2 else 100 * i
        rows.append(f"k_a,1024,{1000 * i},{1000 * i + d}")
    rows.append("k_b,64,0,50")
    csv = tmp_path / "run_kernel_trace.csv"
    csv.write_text("\n".join(rows) + "\n")
    r = subprocess.run([sys.executable, BENCH, "--trace-summary", str(csv), "--skip", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    line = next(l for l in r.stdout.splitlines() if "`k_a`" in l)
    cells = [c.strip() for c in line.strip("|").split("|")]
    assert cells[1:] == ["1,024", "3", "300", "300", "200", "400"], cells
    # a kernel with no more dispatches than the warm-up is summarized over all of them
    line = next(l for l in r.stdout.splitlines() if "`k_b`" in l)
    assert [c.strip() for c in line.strip("|").split("|")][1:] == ["64", "1", "50", "50", "50", "50"]


@pytest.mark.gpu
def test_bench_line_keys(cuda):
    print("bench.py --config c2 --no-others --no-cpu --steps 2 --warmup 1", flush=True)
    r = subprocess.run([sys.executable, BENCH, "--config", "c2", "--no-others", "--no-cpu", "--steps", "2",
                        "--warmup", "1"], capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
    assert len(lines) == 1
    d = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline", "measured_peaks", "cpu_baseline"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 2 and d["warmup"] == 1 and d["dtype"] == "f32"
    assert d["config"]["workload"].startswith("c2:") and d["config"]["global_batch"] == 4_194_304
    assert d["value"] > 0 and abs(d["value"] - 4_194_304 / (d["ms_per_step"] * 1e-3)) < 1e-3 * d["value"]
    rf = d["roofline"]
    assert set(rf) >= {"bound", "achieved", "peak", "unit", "frac", "traffic"}
    assert rf["bound"] == "mfma" and rf["unit"] == "TFLOP/s" and rf["peak"] == 157.3
    assert 0 < rf["frac"] < 1 and abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-3
    mp = d["measured_peaks"]
    assert mp["hbm_copy_GBps"] > 0 and mp["hbm_read_GBps"] > 0 and mp["mfma_f32_TFLOPs"] > 0
    assert abs(mp["frac_of_measured"] - rf["achieved"] / mp["mfma_f32_TFLOPs"]) < 1e-3
