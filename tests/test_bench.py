"""The contract of bench.py's output line: one JSON line on stdout with the
metric, value, unit, step and warm-up counts, dtype, config.workload, and a
roofline object whose fraction follows from its achieved rate and peak and
whose product time fits inside the iteration; more than one GPU is refused
with a message (every box has one MI355X)."""
import contextlib
import io
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
    assert list(d["lines"]) == ["c4_batched_graph_nocopy"]
    assert abs(d["lines"]["c4_batched_graph_nocopy"] - d["value"]) <= 0.01
    # The full line is on stderr.
    full = [json.loads(ln.split("] ", 1)[1]) for ln in r.stderr.splitlines() if ln.startswith("[bench-line] ")]
    assert [ln["name"] for ln in full] == ["c4_batched_graph_nocopy"]


def _harness_record(args):
    """A harness record with every key summarize() reads, numbers carrying
    as many digits as the harness prints."""
    mode, launches, batch, size, rows = args[:5]
    matmul = args[8]
    return {
        "mode": mode, "matmul": matmul, "batch": batch, "size": size, "rows": rows, "copies": 0,
        "launches": launches, "gpu_ms_per_iter": 1.868961, "single_us": 1889.017,
        "submit_us_per_iter": 91.346, "achieved_gbps": 484.8, "valid": 1, "strict_valid": 1,
        "rms_us": 20.001, "rms_gbps": 6714.0, "rms_hbm_frac": 0.8392, "softmax_us": 20.549,
        "softmax_gbps": 6531.7, "softmax_hbm_frac": 0.8165, "matmul_us": 1849.402, "matmul_gbps": 344.7,
        "matmul_tflops": 148.631, "matmul_bound": "mfma", "matmul_frac": 0.9449,
        "rms_max_rel_err": 2.721e-07, "softmax_max_rel_err": 2.8e-07, "product_max_rel_err": 1.885e-07,
        "matmul_within_iter": 1, "one_stream": 0, "host_write": 0, "graph_capture_ms": 0.117605,
        "graph_instantiate_ms": 0.457271, "product_bf16_act_rel_err": 1.234567e-03,
        "warmup_iterations": 57, "min_bytes_per_iter": 805470208, "device": "AMD Instinct MI355X",
    }


def test_full_plan_result_line_fits_the_driver(monkeypatch):
    """The full plan (every harness line, both decoder lines, the four
    lowprec cases, the CPU baseline) prints one stdout line short enough for
    the driver's 8,000-character capture, with every line's microseconds and
    the headline's roofline and cpu_baseline on it; every line in full goes
    to stderr."""
    import bench
    import l2c

    monkeypatch.setattr(l2c, "load_host", lambda: None)
    monkeypatch.setattr(bench, "run_line", lambda lib, args: _harness_record(args))
    monkeypatch.setattr(bench, "run_line_child", lambda lib, args, env: _harness_record(args))
    monkeypatch.setattr(bench, "decoder_line", lambda lib, mode: {
        "name": f"decoder_large_{mode}", "mode": mode, "batch": 1024, "width": 16384, "vocab": 8192, "steps": 4,
        "iterations": 10, "warmup": 3, "compute_us_per_invocation": 7654.321987,
        "compute_single_median_us": 7700.1, "application_us_per_invocation": 7800.2,
        "classifier_tflops_compute_scope": 143.21, "note": "x" * 70})
    monkeypatch.setattr(bench, "lowprec_line", lambda lib, case: {
        "name": f"lowprec_{case}_graph", "mode": "graph", "case": case, "batch": 1024, "width": 16384,
        "vocab": 8192, "steps": 4, "iterations": 10, "warmup": 3, "compute_us_per_invocation": 1111.123456,
        "application_us_per_invocation": 1193.012345, "classifier_flops_per_invocation": 4.398e12,
        "reference_rtx5090_application_us": 1685.8, "speedup_vs_reference": 1.41, "note": "y" * 80})
    cpu = {
        "value": 123456789.123, "unit": "us/iter", "cores": 16, "kind": "port", "sample": "s" * 330,
        "double_oracle": {"value": 98765432.1, "unit": "us/iter", "cores": 1, "sample": "d" * 120},
        "reference_validate_all": {"value": 4567890.12, "unit": "us/call", "cores": 1, "kind": "reference",
                                   "valid": 1, "sample": "r" * 210},
        "measured_s": 12.5,
    }
    monkeypatch.setattr(bench, "cpu_baseline", lambda *a, **k: dict(cpu))
    monkeypatch.setattr(sys, "argv", ["bench.py"])
    out, err = io.StringIO(), io.StringIO()
    with contextlib.redirect_stdout(out), contextlib.redirect_stderr(err):
        assert bench.main() == 0
    printed = [ln for ln in out.getvalue().splitlines() if ln.strip()]
    assert len(printed) == 1
    assert len(printed[0]) <= bench.MAX_STDOUT_LINE, len(printed[0])
    print("result line length", len(printed[0]))
    d = json.loads(printed[0])
    names = ["c4_batched_graph_nocopy"] + [n for n, _ in bench.full_plan(50, 100)] + \
        [n for n, _, _ in bench.child_plan(50, 100)] + \
        ["decoder_large_graph", "decoder_large_direct"] + [f"lowprec_{c}_graph" for c in
                                                           ("fp32", "bf16", "mxfp6", "nvfp4")]
    assert len(names) == len(set(names)) >= 55
    assert list(d["lines"]) == names
    assert d["lines"]["decoder_large_graph"] == 7654.32
    assert d["lines"]["lowprec_nvfp4_graph"] == 1193.01
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "dtype", "config",
                "roofline", "cpu_baseline"):
        assert key in d, key
    assert d["cpu_baseline"]["cores"] == 16 and "measured_s" not in d["cpu_baseline"]
    assert set(d["kernel_fracs"]) >= {"rmsnorm_c4", "softmax_c4", "gemm_f32_c4", "gemv_c2", "scgemm_mxfp4s_c5"}
    full = [json.loads(ln.split("] ", 1)[1]) for ln in err.getvalue().splitlines()
            if ln.startswith("[bench-line] ")]
    assert [ln["name"] for ln in full] == names
