"""Benchmark of the llama2c hot path on one MI355X.

One "step" is one llama2c iteration of the harness (rmsnorm | softmax |
matmul on three streams, joined) over device-resident synthetic inputs. The
headline workload is the largest profiled shape, batch 1024 x dim 16384 x rows
8192, with the batched fp32 contraction on the matrix cores, replayed as a
hipGraph, no copies: `value` is its microseconds per iteration (lower is
better). The other benchmark configurations (decode GEMV 1 x 4096 x 11008,
launch-bound 8 x 768 x 2048, the reference-compatible GEMV iteration at the
large shape, the fused single launch, the MXFP4 / fp8 weights on the bf16
matrix cores and on the block-scaled fp8 matrix cores (MXFP8 activations), and the
loom-private llama2c decoder application at its large shape, and the lowprec
classifier experiment's fp32 / bf16 / MXFP6 / NVFP4 cases at that shape) and
the graph/direct and copy/nocopy splits are each printed in full to stderr as
a "[bench-line] {...}" JSON line; the stdout line carries only their
microseconds ("lines") and the kernels' roofline fractions ("kernel_fracs"),
which keeps it within MAX_STDOUT_LINE characters.

The harness runs in this process (libl2c_host.so via ctypes): HIP events on
each operation's own stream time the kernels, so `roofline` comes from the
same run. cpu_baseline times the oracle's fp32 CPU iteration (llama2.c loop
order, OpenMP over this host's cores) over a bounded sample of the headline
shape and scales it to one whole iteration; the double oracle is timed apart.

Usage: python bench.py [--gpus N] [--steps K] [--warmup W] [--quick]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cuda-elastic_amd"))

HBM_PEAK_GBPS = 8000.0
WARMUP_MS = 100  # the reference harness's default warm-up time (llama2c_cuda_graph.cu:43-53)
FP32_MFMA_PEAK_TFLOPS = 157.3
BF16_MFMA_PEAK_TFLOPS = 2500.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_f32_mfma_c4_traffic.json")
# The result line's length bound: the driver that reads it keeps the last
# 8,000 characters of stdout.
MAX_STDOUT_LINE = 7500


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def run_line(l2c, args):
    t = time.time()
    code, rec, raw = l2c.harness(args)
    log(f"[bench] {' '.join(map(str, args))} -> exit {code} in {time.time() - t:.1f}s: "
        f"gpu_ms_per_iter={rec.get('gpu_ms_per_iter')} valid={rec.get('valid')}")
    if code != 0 or rec.get("valid") != 1:
        raise SystemExit(f"harness run failed (exit {code}): {raw}")
    return rec


def run_line_child(l2c, args, env_overrides):
    """run_line in a child process with extra environment variables: the HIP
    runtime reads settings such as HIP_FORCE_DEV_KERNARG once, at its start."""
    t = time.time()
    env = dict(os.environ, **env_overrides)
    code, rec, raw = l2c.harness(args, in_process=False, env=env, timeout=300)
    log(f"[bench] {' '.join(f'{k}={v}' for k, v in env_overrides.items())} {' '.join(map(str, args))} -> exit "
        f"{code} in {time.time() - t:.1f}s: gpu_ms_per_iter={rec.get('gpu_ms_per_iter')} valid={rec.get('valid')}")
    if code != 0 or rec.get("valid") != 1:
        raise SystemExit(f"harness run failed (exit {code}): {raw[-2000:]}")
    return rec


def summarize(name, rec):
    out = {
        "name": name, "mode": rec["mode"], "matmul": rec["matmul"], "batch": rec["batch"],
        "size": rec["size"], "rows": rec["rows"], "copies": rec["copies"],
        "launches": rec["launches"], "us_per_iter": rec["gpu_ms_per_iter"] * 1000.0,
        "single_us": rec["single_us"], "submit_us_per_iter": rec["submit_us_per_iter"],
        "achieved_gbps": rec["achieved_gbps"], "valid": rec["valid"],
        "strict_valid": rec["strict_valid"],
        "rms_us": rec["rms_us"], "rms_gbps": rec["rms_gbps"], "rms_hbm_frac": rec["rms_hbm_frac"],
        "softmax_us": rec["softmax_us"], "softmax_gbps": rec["softmax_gbps"],
        "softmax_hbm_frac": rec["softmax_hbm_frac"], "matmul_us": rec["matmul_us"],
        "matmul_gbps": rec["matmul_gbps"], "matmul_tflops": rec["matmul_tflops"],
        "matmul_bound": rec["matmul_bound"], "matmul_frac": rec["matmul_frac"],
        "rms_max_rel_err": rec["rms_max_rel_err"], "softmax_max_rel_err": rec["softmax_max_rel_err"],
        "product_max_rel_err": rec["product_max_rel_err"],
        "matmul_within_iter": rec.get("matmul_within_iter"),
        "one_stream": rec.get("one_stream"), "host_write": rec.get("host_write"),
    }
    if rec["matmul"] in ("mxfp4s", "fp8s"):
        # Block-scaled products: matmul_frac is against the 5.0 PFLOP/s dense
        # fp8 matrix peak; the error against the bf16-activation reference is
        # what quantizing the activations to MXFP8 costs (configuration: 2e-3).
        out["product_bf16_act_rel_err"] = rec["product_bf16_act_rel_err"]
    if rec["mode"] == "graph":
        out["graph_capture_ms"] = rec["graph_capture_ms"]
        out["graph_instantiate_ms"] = rec["graph_instantiate_ms"]
    return out


def decoder_line(l2c, mode, iterations=10, warmup=3):
    """The llama2c decoder application at its contract's large shape (1024
    sequences, width 16384, vocab 8192, 4 steps) under the loom_private bench
    protocol; compute scope = token reset + 4 x (rmsnorm, classifier, softmax
    + argmax)."""
    t = time.time()
    code, rec, _ = l2c.decoder(["--action", "bench", "--launch", mode, "--iterations", iterations,
                                "--warmup", warmup], in_process=True)
    if code != 0 or rec is None:
        raise SystemExit(f"decoder bench failed (exit {code})")
    comp, app = rec["timing"]["compute"], rec["timing"]["application"]
    dims = rec["dimensions"]
    flops = 2.0 * dims["classifier_macs_per_step"] * dims["steps"]
    us = comp["batch_per_iteration_us"]
    log(f"[bench] decoder {mode}: compute {us:.1f} us/invocation in {time.time() - t:.1f}s")
    return {"name": f"decoder_large_{mode}", "mode": mode, "batch": dims["batch"], "width": dims["width"],
            "vocab": dims["vocab"], "steps": dims["steps"], "iterations": iterations, "warmup": warmup,
            "compute_us_per_invocation": us, "compute_single_median_us": comp["single_median_us"],
            "application_us_per_invocation": app["batch_per_iteration_us"],
            "classifier_tflops_compute_scope": flops / (us * 1e-6) / 1e12,
            "note": "check-mode parity is a separate run (tests/test_decoder_gpu.py)"}


# Graph application-scope µs per 4-step invocation of the reference's lowprec
# cases on an RTX 5090 (experiments/blackwell/lowprec/README.md:134-139).
LOWPREC_REFERENCE_US = {"fp32": 25285.8, "bf16": 6802.5, "mxfp6": 3816.6, "nvfp4": 1685.8}


def lowprec_line(l2c, case, mode="graph", iterations=10, warmup=3):
    """One case of the lowprec classifier experiment at its primary shape
    (the decoder's large shape with the classifier replaced) under the
    loom_private bench protocol, in-process."""
    t = time.time()
    code, rec, _ = l2c.lowprec(case, ["--action", "bench", "--launch", mode, "--iterations", iterations,
                                      "--warmup", warmup], in_process=True)
    if code != 0 or rec is None:
        raise SystemExit(f"lowprec {case} bench failed (exit {code})")
    comp, app = rec["timing"]["compute"], rec["timing"]["application"]
    dims = rec["dimensions"]
    flops = 2.0 * dims["classifier_macs_per_step"] * dims["steps"]
    us = comp["batch_per_iteration_us"]
    app_us = app["batch_per_iteration_us"]
    log(f"[bench] lowprec {case} {mode}: application {app_us:.1f} us/invocation in {time.time() - t:.1f}s")
    return {"name": f"lowprec_{case}_{mode}", "mode": mode, "case": case, "batch": dims["batch"],
            "width": dims["width"], "vocab": dims["vocab"], "steps": dims["steps"],
            "iterations": iterations, "warmup": warmup,
            "compute_us_per_invocation": us, "application_us_per_invocation": app_us,
            "classifier_flops_per_invocation": flops,
            "reference_rtx5090_application_us": LOWPREC_REFERENCE_US[case],
            "speedup_vs_reference": LOWPREC_REFERENCE_US[case] / app_us,
            "note": "implementation check and accuracy are separate runs (tests/test_lowprec_app_gpu.py)"}


def cpu_threads():
    """The host cores this process may use: its affinity set, capped by
    OMP_NUM_THREADS when set (the GPU boxes set it to the box's CPU share)."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(cap))) if cap.isdigit() and int(cap) > 0 else n


def cpu_baseline(batch, size, rows, sample_vectors, repeats=3):
    """The oracle's fp32 iteration (llama2.c loop order) on the host's cores
    (OpenMP over rows and vectors): rmsnorm and softmax of every vector and
    the product of sample_vectors of them against all rows, each the median
    of `repeats` runs, the product scaled linearly to the whole batch (every
    vector costs the same; the bench passes the whole batch, about 10-15 s of
    host time over the three runs). The double oracle (the validation
    reference) is timed apart on one thread."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle

    L = oracle.lib()
    threads = cpu_threads()
    t_start = time.perf_counter()
    inp = oracle.fill("scaled", 1, batch, size, rows)
    n = np.empty(batch * size, np.float32)
    s = np.empty(batch * size, np.float32)
    p = np.empty(batch * rows, np.float32)

    def median_time(fn):
        times = []
        for _ in range(repeats):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return sorted(times)[len(times) // 2]

    t_vec = median_time(lambda: L.orc_iteration_f32_mt(inp.input, inp.probabilities, inp.weight, inp.matrix,
                                                         batch, size, 0, 1, 0, n, s, p, threads))
    t_mm = median_time(lambda: L.orc_iteration_f32_mt(inp.input, inp.probabilities, inp.weight, inp.matrix,
                                                        0, size, rows, 1, sample_vectors, n, s, p, threads))
    per_iter_s = t_vec + t_mm * batch / sample_vectors
    # Double oracle: the product reference and tolerance of 4 vectors.
    dv = 4
    t0 = time.perf_counter()
    oracle.product_check(False, True, inp.input, inp.matrix, p, batch, size, rows, list(range(dv)))
    t_dbl = time.perf_counter() - t0
    ref = reference_validate_all(inp, n, s, p, batch, size, rows)
    return {
        "value": per_iter_s * 1e6, "unit": "us/iter", "cores": threads, "kind": "port",
        "sample": (f"oracle orc_iteration_f32_mt (fp32, llama2.c loop order, {threads} OpenMP threads): "
                   f"rmsnorm+softmax of all {batch} vectors ({t_vec:.3f} s) and the product of "
                   f"{sample_vectors} of {batch} vectors x {rows} rows x {size} ({t_mm:.2f} s), medians "
                   f"of {repeats}" + ("" if sample_vectors == batch else
                                      f", the product scaled linearly to one {batch}x{size}x{rows} iteration")),
        "double_oracle": {
            "value": t_dbl * batch / dv * 1e6, "unit": "us/iter", "cores": 1,
            "sample": f"orc_product_check (double reference + tolerance) of {dv} vectors x {rows} rows x "
                      f"{size} ({t_dbl:.2f} s), scaled to {batch} vectors"},
        "reference_validate_all": ref,
        "measured_s": time.perf_counter() - t_start,
    }


def reference_validate_all(inp, normalized, softmax, product, batch, size, rows):
    """The reference's own CPU code, validate_all (llama2c/llama2c_common.h:
    231-319: the double rmsnorm and softmax references over every vector and
    the double product reference with its gamma bound over every row), as
    compiled from the reference's sources into oracle/_ref/libl2c_ref.so,
    timed once on one thread on the legacy iteration's outputs at this shape
    (the product of vector 0). None when that library was not built."""
    import numpy as np
    import oracle
    try:
        R = oracle.ref()
    except (OSError, AttributeError) as e:
        R, why = None, str(e)
    else:
        why = "oracle/_ref/libl2c_ref.so was not built"
    if R is None:
        log(f"[bench] the reference's validate_all not timed: {why}")
        return None
    tol = np.empty(rows, np.float32)
    refv = np.empty(rows, np.float64)
    # The legacy iteration's product is W . x[0]; the batched product's first
    # row holds exactly that vector's outputs.
    p0 = np.ascontiguousarray(product[:rows])
    t0 = time.perf_counter()
    valid = R.ref_validate_all(1, 1, inp.input, inp.probabilities, inp.weight, inp.matrix, normalized,
                               softmax, p0, batch, size, rows, tol, refv)
    t = time.perf_counter() - t0
    return {"value": t * 1e6, "unit": "us/call", "cores": 1, "kind": "reference", "valid": int(valid),
            "sample": (f"the reference's validate_all (double rmsnorm + softmax references of {batch} x {size}, "
                       f"double product reference + gamma bound of {rows} rows x {size}) on the oracle's "
                       f"fp32 outputs, one call, one thread")}


B_C4, S_C4, R_C4 = 1024, 16384, 8192


def plan_args(mode, launches, batch, size, rows, copies, matmul, inputs="scaled=1", warm=100, extra=()):
    """The harness argv of one bench line (the reference CLI's positional
    order, llama2c_cuda_graph.cu:195-258, plus this build's keyword tokens)."""
    return [mode, launches, batch, size, rows, 1, WARMUP_MS, copies, matmul, inputs,
            f"warmup_iters={warm}", *extra]


def full_plan(K, W):
    """(name, argv) of every harness line after the headline: the C1 smoke
    shape, the graph / direct and copy / nocopy splits of C2, C3 and C4, the
    fused launch, the one-stream and host-write iteration forms, and the four
    C5 formats."""
    B, S, R = B_C4, S_C4, R_C4
    c2 = (1, 4096, 11008)
    c3 = (8, 768, 2048)

    def cfg(mode, launches, shape, copies, matmul, inputs="scaled=1", warm=W, extra=()):
        return plan_args(mode, launches, *shape, copies, matmul, inputs=inputs, warm=warm, extra=extra)

    c4 = (B, S, R)
    c1 = (1, 288, 288)
    plan = [
        ("c1_graph_nocopy", cfg("graph", 10000, c1, "nocopy", "coalesced", warm=100)),
        ("c1_direct_nocopy", cfg("direct", 10000, c1, "nocopy", "coalesced", warm=100)),
        ("c1_fused_direct_nocopy", cfg("direct", 10000, c1, "nocopy", "fused", warm=100)),
        ("c4_batched_direct_nocopy", cfg("direct", K, c4, "nocopy", "batched")),
        ("c4_batched_graph_copy", cfg("graph", K, c4, "copy", "batched")),
        ("c4_batched_direct_copy", cfg("direct", K, c4, "copy", "batched")),
        ("c4_gemv_graph_nocopy", cfg("graph", 200, c4, "nocopy", "coalesced")),
        ("c4_gemv_direct_nocopy", cfg("direct", 200, c4, "nocopy", "coalesced")),
        ("c4_fused_graph_nocopy", cfg("graph", 200, c4, "nocopy", "fused")),
        ("c4_fused_direct_nocopy", cfg("direct", 200, c4, "nocopy", "fused")),
        ("c2_gemv_graph_nocopy", cfg("graph", 1000, c2, "nocopy", "coalesced", warm=50)),
        ("c2_gemv_direct_nocopy", cfg("direct", 1000, c2, "nocopy", "coalesced", warm=50)),
        ("c2_fused_graph_nocopy", cfg("graph", 1000, c2, "nocopy", "fused", warm=50)),
        ("c2_fused_direct_nocopy", cfg("direct", 1000, c2, "nocopy", "fused", warm=50)),
        ("c3_graph_nocopy", cfg("graph", 10000, c3, "nocopy", "coalesced", warm=100)),
        ("c3_direct_nocopy", cfg("direct", 10000, c3, "nocopy", "coalesced", warm=100)),
        ("c3_graph_copy", cfg("graph", 10000, c3, "copy", "coalesced", warm=100)),
        ("c3_direct_copy", cfg("direct", 10000, c3, "copy", "coalesced", warm=100)),
        ("c3_fused_graph_nocopy", cfg("graph", 10000, c3, "nocopy", "fused", warm=100)),
        ("c3_fused_direct_nocopy", cfg("direct", 10000, c3, "nocopy", "fused", warm=100)),
        ("c3_fused_direct_copy", cfg("direct", 10000, c3, "copy", "fused", warm=100)),
    ]
    # Iteration forms beyond the reference protocol: one stream without
    # fork/join events, and copy-mode downloads by device stores into the
    # pinned host buffers (hostwrite) in place of memcpy nodes / calls.
    plan += [
        ("c3_onestream_graph_nocopy", cfg("graph", 10000, c3, "nocopy", "coalesced", warm=100, extra=("onestream",))),
        ("c3_onestream_direct_nocopy", cfg("direct", 10000, c3, "nocopy", "coalesced", warm=100,
                                           extra=("onestream",))),
        ("c3_onestream_graph_copy", cfg("graph", 10000, c3, "copy", "coalesced", warm=100, extra=("onestream",))),
        ("c3_graph_copy_hostwrite", cfg("graph", 10000, c3, "copy", "coalesced", warm=100, extra=("hostwrite",))),
        ("c3_direct_copy_hostwrite", cfg("direct", 10000, c3, "copy", "coalesced", warm=100, extra=("hostwrite",))),
        ("c2_onestream_graph_nocopy", cfg("graph", 1000, c2, "nocopy", "coalesced", warm=50, extra=("onestream",))),
        ("c2_onestream_direct_nocopy", cfg("direct", 1000, c2, "nocopy", "coalesced", warm=50, extra=("onestream",))),
        ("c4_batched_graph_copy_hostwrite", cfg("graph", K, c4, "copy", "batched", extra=("hostwrite",))),
        ("c4_batched_direct_copy_hostwrite", cfg("direct", K, c4, "copy", "batched", extra=("hostwrite",))),
        ("c4_batched_onestream_graph_nocopy", cfg("graph", K, c4, "nocopy", "batched", extra=("onestream",))),
    ]
    for fmt in ("mxfp4", "fp8", "mxfp4s", "fp8s"):
        for mode in ("graph", "direct"):
            for copies in ("nocopy", "copy"):
                plan.append((f"c5_{fmt}_{mode}_{copies}", cfg(mode, K, c4, copies, fmt, inputs="normal=1")))
        plan.append((f"c5_{fmt}_onestream_graph_nocopy",
                     cfg("graph", K, c4, "nocopy", fmt, inputs="normal=1", extra=("onestream",))))
    return plan


# C3 lines with the kernel arguments left in host memory (HIP_FORCE_DEV_KERNARG=0,
# a process-wide HIP runtime setting): the three-stream graph replay then runs
# faster than direct launches; every other line keeps the runtime's default.
HOST_KERNARG = {"HIP_FORCE_DEV_KERNARG": "0"}


def child_plan(K, W):
    """(name, argv, environment) of the lines that run in a child process."""
    c3 = (8, 768, 2048)
    return [
        ("c3_graph_nocopy_hostkernarg", plan_args("graph", 10000, *c3, "nocopy", "coalesced", warm=100), HOST_KERNARG),
        ("c3_direct_nocopy_hostkernarg", plan_args("direct", 10000, *c3, "nocopy", "coalesced", warm=100), HOST_KERNARG),
    ]


def emit(line):
    """Prints one bench line in full to stderr, as its own short JSON line,
    and returns it; stdout carries only the compact summary of all lines."""
    log("[bench-line] " + json.dumps(line, separators=(",", ":")))
    return line


def line_us(line):
    """The microseconds a line is summarized by on stdout: the iteration for
    harness lines, the compute scope per invocation for the decoder and the
    application scope per invocation for lowprec lines."""
    if "us_per_iter" in line:
        return line["us_per_iter"]
    if line["name"].startswith("lowprec_"):
        return line["application_us_per_invocation"]
    return line["compute_us_per_invocation"]


def kernel_fractions(lines):
    """Roofline fractions of each kernel, from the first line that times it
    alone: rmsnorm / softmax / matrix-vector product against 8 TB/s of HBM,
    the fp32 contraction against 157.3 TF, the exact C5 contractions against
    2.5 PF bf16 and the block-scaled ones against 5.0 PF fp8."""
    pick = {
        "rmsnorm_c4": ("c4_batched_graph_nocopy", "rms_hbm_frac"),
        "softmax_c4": ("c4_batched_graph_nocopy", "softmax_hbm_frac"),
        "gemm_f32_c4": ("c4_batched_graph_nocopy", "matmul_frac"),
        "gemv_c4": ("c4_gemv_graph_nocopy", "matmul_frac"),
        "gemv_c2": ("c2_gemv_graph_nocopy", "matmul_frac"),
        "qgemm_mxfp4_c5": ("c5_mxfp4_graph_nocopy", "matmul_frac"),
        "qgemm_fp8_c5": ("c5_fp8_graph_nocopy", "matmul_frac"),
        "scgemm_mxfp4s_c5": ("c5_mxfp4s_graph_nocopy", "matmul_frac"),
        "scgemm_fp8s_c5": ("c5_fp8s_graph_nocopy", "matmul_frac"),
    }
    by_name = {ln["name"]: ln for ln in lines}
    out = {}
    for key, (name, field) in pick.items():
        if name in by_name and by_name[name].get(field) is not None:
            out[key] = round(by_name[name][field], 4)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # Warm-up: at least W iterations and at least the reference protocol's
    # default 100 ms (llama2c_cuda_graph.cu:43-53,409-431), whichever is
    # longer; a few iterations alone leave the clocks ramping through the
    # timed loop (its first ~30 ms run up to 12% slow at the headline shape).
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--quick", action="store_true", help="headline and cpu baseline only")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported on this build "
              "(every GPU box has one MI355X; the path would shard W and the output rows across GPUs, "
              "one all-gather of outputs being the only exchange)",
              file=sys.stderr)
        return 2
    import l2c

    l2c.load_host()
    K, W = args.steps, args.warmup
    B, S, R = B_C4, S_C4, R_C4

    headline = run_line(l2c, plan_args("graph", K, B, S, R, "nocopy", "batched", warm=W))
    lines = [emit(summarize("c4_batched_graph_nocopy", headline))]
    if not args.quick:
        for name, a in full_plan(K, W):
            lines.append(emit(summarize(name, run_line(l2c, a))))
        for name, a, env in child_plan(K, W):
            line = summarize(name, run_line_child(l2c, a, env))
            line["env"] = env
            lines.append(emit(line))
        for mode in ("graph", "direct"):
            lines.append(emit(decoder_line(l2c, mode)))
        for case in ("fp32", "bf16", "mxfp6", "nvfp4"):
            lines.append(emit(lowprec_line(l2c, case)))

    gemm_us = headline["matmul_us"]
    flops = 2.0 * B * R * S
    achieved = flops / (gemm_us * 1e-6) / 1e12
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        try:
            traffic = json.load(open(TRAFFIC_FILE)).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    consistent = gemm_us <= headline["gpu_ms_per_iter"] * 1000.0
    if not consistent:
        log(f"[bench] WARNING: the product alone ({gemm_us:.1f} us) exceeds the iteration that contains it "
            f"({headline['gpu_ms_per_iter'] * 1000.0:.1f} us)")
    roofline = {
        "kernel": "gemm_f32_mfma_kernel (l2c_matmul, v_mfma_f32_32x32x2_f32)",
        "bound": "mfma", "achieved": achieved, "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
        "frac": achieved / FP32_MFMA_PEAK_TFLOPS, "traffic": traffic,
        "algorithmic_flops_per_launch": flops,
        "avg_launch_us": gemm_us,
        "within_iteration": consistent,
        "timing": ("HIP events on the matmul stream: l2c_matmul alone, back to back for >= 100 ms, then the "
                   "median of 5 back-to-back windows of K launches"),
    }
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(B, S, R, sample_vectors=B)
        log(f"[bench] cpu baseline {cpu['value'] / 1e6:.1f} s/iter ({cpu['measured_s']:.1f} s measured)")
        cpu.pop("measured_s")
    us = headline["gpu_ms_per_iter"] * 1000.0
    result = {
        "metric": "us/iter (llama2c iteration: rmsnorm + softmax + batched fp32 W.x on MFMA), hipGraph",
        "value": us, "unit": "us/iter", "n_gpus": 1, "steps": headline["launches"], "warmup": W,
        "warmup_protocol": {"min_iterations": W, "min_ms": WARMUP_MS,
                            "iterations_run": headline["warmup_iterations"]},
        "ms_per_step": headline["gpu_ms_per_iter"], "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: seeded splitmix64 inputs, scaled distributions (x,logits U[-1,1), "
                "weight U[0.5,1.5), W U[-1/128,1/128)), device-resident",
        "config": {"workload": "C4 llama2c iteration, batch 1024 x dim 16384 x rows 8192, batched "
                               "fp32 matmul on matrix cores, hipGraph replay, no copies",
                   "batch": B, "size": S, "rows": R, "mode": "graph", "copies": 0,
                   "matmul": "batched", "iteration_flops": flops,
                   "iteration_min_bytes": headline["min_bytes_per_iter"]},
        "tflops": headline["matmul_tflops"],
        "rms_gbps": headline["rms_gbps"], "softmax_gbps": headline["softmax_gbps"],
        "roofline": roofline,
        "cpu_baseline": cpu,
        # Every line in full is on stderr ("[bench-line] {...}"); here only its
        # microseconds (iteration, or invocation for decoder / lowprec lines)
        # and each kernel's roofline fraction, so the line stays short.
        "lines": {ln["name"]: round(line_us(ln), 2) for ln in lines},
        "kernel_fracs": kernel_fractions(lines),
        "device": headline.get("device"),
    }
    text = json.dumps(result)
    if len(text) > MAX_STDOUT_LINE:
        # Keep the headline, roofline and cpu baseline readable: the per-line
        # microseconds are on stderr anyway.
        log(f"[bench] WARNING: result line of {len(text)} characters; dropping the lines map from stdout")
        result["lines"] = {"c4_batched_graph_nocopy": result["lines"]["c4_batched_graph_nocopy"]}
        text = json.dumps(result)
    print(text, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
