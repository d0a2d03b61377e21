"""The sweep tooling (l2c.sweep): config grammar, CSV columns and the derived
speedup metrics of the reference's plot_sweep.py:29-73, on a synthetic CSV
whose ratios are known (CPU); a two-config sweep on the GPU."""
import csv
import math

import pytest

from l2c import sweep


def test_parse_config():
    assert sweep.parse_config("1,16,16") == (1, 16, 16, 1, "copy")
    assert sweep.parse_config("1024,256,8192,8,nocopy") == (1024, 256, 8192, 8, "nocopy")
    with pytest.raises(ValueError):
        sweep.parse_config("1,2")
    with pytest.raises(ValueError):
        sweep.parse_config("1,2,3,1,sometimes")


def test_reference_config_sets():
    # profile_cuda.sh:107-124: 9 launch-overhead configs, 10 GPU-filling configs.
    assert len(sweep.SWEEP_CONFIGS.split()) == 9 and len(sweep.FILL_CONFIGS.split()) == 10
    for c in sweep.SWEEP_CONFIGS.split() + sweep.FILL_CONFIGS.split():
        sweep.parse_config(c)


def _row(trial, mode, gpu, wall, submit, setup=(0.0, 0.0, 0.0), valid=1, code=0, batch=1):
    r = dict.fromkeys(sweep.HEADER, "")
    r.update(trial=trial, mode=mode, launches=30, batch=batch, size=16, rows=16, repeats=1,
             copies="nocopy", matmul="naive", warmup_ms=100, gpu_ms_per_iter=gpu,
             wall_ms_per_iter=wall, submit_us_per_iter=submit, graph_capture_ms=setup[0],
             graph_instantiate_ms=setup[1], graph_upload_ms=setup[2], min_waves=0.5,
             achieved_gbps=10, valid=valid, exit_code=code)
    return r


def test_speedup_metrics(tmp_path):
    path = tmp_path / "sweep-x.csv"
    rows = [
        _row(1, "direct", 4.0, 4.5, 3.0), _row(1, "graph", 2.0, 2.5, 1.5, (0.5, 0.25, 0.25)),
        _row(2, "graph", 2.0, 2.5, 1.0, (0.5, 0.25, 0.25)), _row(2, "direct", 3.0, 3.5, 3.0),
        # an invalid run and a failed run are ignored
        _row(3, "direct", 1.0, 1.0, 1.0, valid=0), _row(3, "graph", 9.0, 9.0, 9.0, code=1),
        # a config with only one mode has no pair
        _row(1, "direct", 1.0, 1.0, 1.0, batch=2),
    ]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=sweep.HEADER)
        w.writeheader()
        w.writerows(rows)
    out = sweep.speedup_rows(str(path))
    assert len(out) == 1
    r = out[0]
    assert r["trials"] == 2
    assert math.isclose(r["gpu_speedup"], (2.0 + 1.5) / 2)
    assert r["gpu_speedup_min"] == 1.5 and r["gpu_speedup_max"] == 2.0
    assert math.isclose(r["submit_speedup"], (2.0 + 3.0) / 2)
    assert math.isclose(r["graph_setup_ms"], 1.0)
    # wall saving per replay = mean(4.5, 3.5) - mean(2.5, 2.5) = 1.5 ms -> ceil(1.0 / 1.5) = 1
    assert r["break_even_replays"] == 1
    out_path, _ = sweep.write_speedup(str(path))
    assert out_path.endswith("sweep-x-speedup.csv")
    with open(out_path) as f:
        assert f.readline().startswith("batch,size,rows,repeats,copies,matmul,trials,")


@pytest.mark.gpu
def test_small_sweep_on_gpu(torch_gpu, tmp_path):
    print("case sweep 2 configs x 1 trial", flush=True)
    path = sweep.run_sweep("sweep", "1,64,64,1,nocopy 8,768,2048,2,copy", "20", "coalesced", trials=1,
                           warmup_ms=20, out_dir=str(tmp_path), timeout=120)
    with open(path) as f:
        rows = list(csv.DictReader(f))
    assert len(rows) == 4
    assert all(r["exit_code"] == "0" and r["valid"] == "1" for r in rows)
    assert [r["mode"] for r in rows] == ["direct", "graph", "direct", "graph"]
    _, summary = sweep.write_speedup(path)
    assert len(summary) == 2 and all(s["gpu_speedup"] > 0 for s in summary)


def test_check_and_compare_plans():
    """The run plans restate the reference's matrices: check = 3 shapes x
    {deterministic, random=1, random=2} x 4 variants x graph/direct x
    copy/nocopy (llama2c/Makefile:44-56); compare = one group of graph /
    direct / fused / naive runs per shape x input set (compare_sota.sh:41-71)."""
    from l2c import matrix
    plan = matrix.check_plan()
    assert len(plan) == 3 * 3 * 4 * 2 * 2 and len(set(plan)) == len(plan)
    assert {(c.batch, c.size, c.rows, c.repeats) for c in plan} == set(matrix.CHECK_SHAPES)
    assert {c.variant for c in plan} == {"coalesced", "naive", "fused", "batched"}
    assert plan[0].argv() == ["graph", "auto", "64", "1000", "300", "1", "1", "nocopy", "coalesced",
                              "deterministic"]
    groups = matrix.compare_plan()
    assert len(groups) == 3 * 4
    for g in groups:
        assert [c.label for c in g] == ["graph", "direct", "fused", "naive"]
        assert len({(c.batch, c.size, c.rows, c.inputs, c.copies) for c in g}) == 1
    assert groups[0][0].argv("/tmp/x.bin")[-1] == "--dump=/tmp/x.bin"


def test_launch_trace_summary_on_a_synthetic_trace(tmp_path):
    """l2c.launch_trace on a trace whose figures are known: 8 graph launches
    of 20 us host time each, one 3 us kernel per launch starting 5 us after
    the call returns, one launch every 20 us."""
    from l2c import launch_trace

    api, kernels = [], []
    for i in range(8):
        t0 = 1_000_000 + i * 20_000
        api.append({"Function": "hipGraphLaunch", "Correlation_Id": str(i), "Start_Timestamp": str(t0),
                    "End_Timestamp": str(t0 + 20_000)})
        k0 = t0 + 25_000
        kernels.append({"Kernel_Name": "fused_kernel", "Correlation_Id": str(i), "Start_Timestamp": str(k0),
                        "End_Timestamp": str(k0 + 3_000)})
    d = tmp_path / "trace" / "host"
    d.mkdir(parents=True)
    for name, rows in (("t_hip_api_trace.csv", api), ("t_kernel_trace.csv", kernels)):
        with open(d / name, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=list(rows[0]))
            w.writeheader()
            w.writerows(rows)
    s = launch_trace.summarize_dir(str(tmp_path / "trace"))
    assert s["api"]["hipGraphLaunch"] == {"n": 8, "mean_us": 20.0, "median_us": 20.0}
    assert s["kernels"]["fused_kernel"] == {"n": 8, "mean_us": 3.0}
    assert s["steady"]["kernels"] == 4 and s["steady"]["gap_median_us"] == 17.0
    assert s["steady"]["busy_frac"] == round(12.0 / 63.0, 3)
    assert s["call_end_to_kernel_start_us"]["hipGraphLaunch"]["median"] == 5.0


def test_overlap_summary_on_a_synthetic_trace(tmp_path):
    """l2c.overlap on a trace whose figures are known: 8 iterations 130 us
    apart, a 100 us product, rmsnorm inside it (+5 .. +45 us) and softmax
    after it (+100 .. +125 us, so it belongs to the gap before the next
    product)."""
    from l2c import overlap

    kernels = []
    for i in range(8):
        p0 = 1_000_000 + i * 130_000
        kernels.append({"Kernel_Name": "scaled_gemm_wide_kernel(float*)", "Start_Timestamp": str(p0),
                        "End_Timestamp": str(p0 + 100_000)})
        kernels.append({"Kernel_Name": "rmsnorm_kernel<8>", "Start_Timestamp": str(p0 + 5_000),
                        "End_Timestamp": str(p0 + 45_000)})
        kernels.append({"Kernel_Name": "softmax_kernel<8>", "Start_Timestamp": str(p0 + 100_000),
                        "End_Timestamp": str(p0 + 125_000)})
    d = tmp_path / "trace" / "host"
    d.mkdir(parents=True)
    with open(d / "t_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(kernels[0]))
        w.writeheader()
        w.writerows(kernels)
    # The harness also times the product alone: 4 launches back to back, no rows.
    p0 = 1_000_000 + 8 * 130_000 + 50_000
    for i in range(4):
        kernels.append({"Kernel_Name": "scaled_gemm_wide_kernel(float*)", "Start_Timestamp": str(p0 + i * 100_000),
                        "End_Timestamp": str(p0 + (i + 1) * 100_000)})
    with open(d / "t_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(kernels[0]))
        w.writeheader()
        w.writerows(kernels)
    s = overlap.summarize_dir(str(tmp_path / "trace"), "scaled_gemm_wide", ["rmsnorm", "softmax"])
    assert s["launches"] == 12 and s["iterations"] == 8 and s["steady_iterations"] == 4
    assert s["product_us"] == 100.0 and s["gap_us"] == 30.0 and s["period_us"] == 130.0
    assert s["rows"]["rmsnorm"] == {"n": 4, "start_us": 5.0, "end_us": 45.0, "inside_product": 1.0}
    assert s["rows"]["softmax"] == {"n": 4, "start_us": -30.0, "end_us": -5.0, "inside_product": 0.0}


def test_power_parsers():
    """l2c.power reads amd-smi's socket power, rocm-smi's shader clock and the
    kernel bench's result line as those tools print them on MI355X."""
    from l2c import power
    amd = "GPU: 0\n    POWER:\n        SOCKET_POWER: 1310 W\n        GFX_VOLTAGE: N/A\n"
    assert power.parse_socket_power(amd) == 1310.0
    assert power.parse_socket_power("GPU: 0\n    POWER:\n        SOCKET_POWER: N/A\n") is None
    smi = "==== Current clock frequencies ====\nGPU[0]\t\t: sclk clock level: 1: (1963Mhz)\n"
    assert power.parse_sclk(smi) == 1963.0
    assert power.parse_sclk("GPU[0]\t\t: sclk clock level: S: (95Mhz)") == 95.0
    line = ("op=fp8s batch=1024 size=16384 rows=8192 iters=30000 warmup=608 avg_us=126.760 "
            "bytes=201359360 gbps=1588.5 tflops=2168.491")
    rec = power.parse_result(line)
    assert rec["op"] == "fp8s" and rec["avg_us"] == 126.76 and rec["iters"] == 30000.0
