"""The profiling tool the profile summaries' commands run, bin/l2c_kernel_bench:
every op runs on a small shape and prints its result line, the vendor GEMMs
it times for comparison agree with this library's contraction, and the
register-only MFMA loops report rates that do not exceed the datasheet
peaks (llama2c/profile_cuda.sh:136-167 isolates kernels the same way)."""
import os
import re
import subprocess

import pytest

from conftest import PKG

pytestmark = pytest.mark.gpu

BENCH = os.path.join(PKG, "bin", "l2c_kernel_bench")
SHAPE = (256, 1024, 512)  # batch, size (k), rows: every op's divisibility holds
OPS = ["rmsnorm", "softmax", "gemv", "naive", "fused", "matmul", "mxfp4", "fp8", "mxfp4s", "mxfp4s_narrow", "fp8s",
       "cvt_mxfp8", "bf16", "mxfp6", "cvt_bf16", "cvt_mxfp6", "cvt_nvfp4", "copy", "gemv_cold", "gemv_cold_copy",
       "read_cold", "rmsnorm_cold", "softmax_cold", "copy_cold", "read", "vendor_f32", "vendor_bf16",
       "stage_wstep", "stage_wpair", "stage_split64", "stage_split128", "stage_fp8", "mfma_f8f4",
       "mfma_f8f8", "mfma_bf16"]


def run(*args, timeout=180):
    print("case l2c_kernel_bench", " ".join(map(str, args)), flush=True)
    return subprocess.run([BENCH, *map(str, args)], capture_output=True, text=True, timeout=timeout)


@pytest.mark.parametrize("op", OPS)
def test_op_runs(torch_gpu, op):
    r = run(op, *SHAPE, 3)
    assert r.returncode == 0, r.stderr
    line = r.stdout.strip().splitlines()[-1]
    assert line.startswith(f"op={op} batch={SHAPE[0]} size={SHAPE[1]} rows={SHAPE[2]} "), line
    assert float(re.search(r"avg_us=([0-9.]+)", line).group(1)) > 0.0
    if op.endswith("_cold") or op == "gemv_cold_copy":
        assert ("flush=copy_512MiB" if op == "gemv_cold_copy" else "flush=read_1GiB") in line


@pytest.mark.parametrize("op", ["vendor_f32", "vendor_bf16"])
def test_vendor_gemm_matches_the_contraction(torch_gpu, op):
    # hipBLASLt's result against l2c_matmul / l2c_matmul_bf16 over every
    # output, relative to the largest output: both accumulate in fp32 over
    # k = 1024, in different orders.
    r = run(op, *SHAPE, 3)
    assert r.returncode == 0, r.stderr
    m = re.search(r"vendor_check max_rel_diff=([0-9.eE+-]+)", r.stdout)
    assert m, r.stdout
    assert float(m.group(1)) < 1e-5
    assert re.search(r"vendor_pick=\d+ of \d+", r.stdout)


DATASHEET_TFLOPS = {"fp32": 157.3, "bf16": 2500.0, "fp6": 10100.0, "fp8": 5000.0}


def test_mfma_ceilings(torch_gpu):
    r = run("ceiling", timeout=300)
    assert r.returncode == 0, r.stderr
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("ceiling mfma=")]
    assert len(lines) == 9, r.stdout  # six 32 x 32 (and fp32 16 x 16) loops, three 16 x 16 ones
    for ln in lines:
        rates = {k: float(v) for k, v in re.findall(r"(\w+_tflops)=([0-9.]+)", ln)}
        assert set(rates) == {"constant_tflops", "random_tflops", "random_one_wave_tflops"}, ln
        peak = DATASHEET_TFLOPS[re.search(r"mfma=(fp32|bf16|fp6|fp8)", ln).group(1)]
        # The datasheet peaks assume 2.4 GHz, the top engine clock.
        assert 0.0 < rates["random_tflops"] <= rates["constant_tflops"] * 1.02, ln
        assert 0.5 * peak < rates["constant_tflops"] <= 1.02 * peak, ln
        assert 0.0 < rates["random_one_wave_tflops"] <= 1.02 * peak, ln


def test_lds_read_rates(torch_gpu):
    # Six lines (b128 / b64 at 4, 8, 16 waves a CU); a rate in bytes per shader
    # clock per CU that grows with the waves in flight and stays under 512 B/clk,
    # and a shader clock within the part's range.
    r = run("lds", timeout=120)
    assert r.returncode == 0, r.stderr
    rates = {}
    for read, waves, rate, ghz in re.findall(
            r"lds read=(b128|b64) waves_per_cu=(\d+) bytes_per_clk_per_cu=([0-9.]+) clock_ghz=([0-9.]+)", r.stdout):
        rates[(read, int(waves))] = float(rate)
        assert 0.5 < float(ghz) < 2.6, r.stdout
    assert len(rates) == 6, r.stdout
    for read in ("b128", "b64"):
        assert 0.0 < rates[(read, 4)] < rates[(read, 16)] < 512.0, rates
