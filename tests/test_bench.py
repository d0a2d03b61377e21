"""The contract of bench.py's output line: one JSON line on stdout with the
metric, value, unit, step and warm-up counts, dtype, config.workload, and a
roofline object whose fraction follows from its achieved rate and peak and
whose product time fits inside the iteration; more than one GPU is refused
with a message (every box has one MI355X)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout.strip() == ""


@pytest.mark.gpu
def test_quick_bench_line(torch_gpu):
    print("case bench.py --quick --no-cpu --steps 3 --warmup 2", flush=True)
    r = subprocess.run([sys.executable, "-u", BENCH, "--quick", "--no-cpu", "--steps", "3", "--warmup", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1, r.stdout
    d = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline", "lines"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["warmup"] == 2
    assert d["unit"] == "us/iter" and d["higher_is_better"] is False and d["dtype"] == "f32"
    assert d["value"] > 0 and abs(d["ms_per_step"] * 1000.0 - d["value"]) <= 1e-6 * d["value"]
    assert d["config"]["workload"].startswith("C4 llama2c iteration")
    assert (d["config"]["batch"], d["config"]["size"], d["config"]["rows"]) == (1024, 16384, 8192)
    roof = d["roofline"]
    assert roof["bound"] == "mfma" and roof["unit"] == "TFLOP/s" and roof["peak"] == 157.3
    assert 0.0 < roof["frac"] <= 1.0
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) <= 1e-9
    # The product's launch time, measured alone, fits in the iteration that contains it.
    assert roof["within_iteration"] is True and roof["avg_launch_us"] <= d["value"]
    assert d["cpu_baseline"] is None  # --no-cpu
    assert [ln["name"] for ln in d["lines"]] == ["c4_batched_graph_nocopy"]
