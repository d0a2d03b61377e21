"""Socket power and shader clock while one operation runs back to back.

For each `OP:ITERS` it starts `bin/l2c_kernel_bench OP BATCH SIZE ROWS ITERS`
(ITERS chosen so the run lasts a few seconds), or for `--harness "ARGS"` the
harness `bin/llama2c_hip ARGS` (its time is gpu_ms_per_iter), waits past the
tool's warm-up,
then reads the socket power (`amd-smi metric -p`, SOCKET_POWER) and the
current shader clock (`rocm-smi -c`, the sclk line) a few times while the
operation is still running, and finally the tool's own result line. The idle
power is read once before the first operation, after the device has had
`--idle-settle` seconds without work.

    python -m l2c.power fp8s:30000 mxfp4s:35000 stage_fp8:60000 matmul:2000 [--shape 1024 16384 8192]
                        [--harness "graph 30000 1024 16384 8192 1 100 nocopy mxfp4s normal=1" ...]
                        [--settle 2.0] [--samples 3] [--idle-settle 8.0] [--out FILE.json]

Power and clock tell whether a kernel runs at the device's power limit (the
clock drops below its maximum while the socket power sits near the cap) or at
full clock; with the kernel's time they give its energy per launch.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(PKG, "bin", "l2c_kernel_bench")
HARNESS = os.path.join(PKG, "bin", "llama2c_hip")


def parse_socket_power(text: str) -> float | None:
    """Watts from `amd-smi metric -p` output (the first SOCKET_POWER line)."""
    m = re.search(r"SOCKET_POWER:\s*([0-9.]+)\s*W", text)
    return float(m.group(1)) if m else None


def parse_sclk(text: str) -> float | None:
    """MHz of the current shader clock level from `rocm-smi -c` output."""
    m = re.search(r"sclk clock level:\s*\S+\s*\(([0-9.]+)\s*Mhz\)", text, re.IGNORECASE)
    return float(m.group(1)) if m else None


def parse_result(line: str) -> dict:
    """key=value fields of l2c_kernel_bench's result line (numbers as floats)."""
    out = {}
    for key, value in re.findall(r"(\w+)=(\S+)", line):
        try:
            out[key] = float(value)
        except ValueError:
            out[key] = value
    return out


def _read(cmd: list[str]) -> str:
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=30)
    return r.stdout + r.stderr


def sample() -> tuple[float | None, float | None]:
    return parse_socket_power(_read(["amd-smi", "metric", "-p"])), parse_sclk(_read(["rocm-smi", "-c"]))


def measure(op: str, iters: int, shape: tuple[int, int, int], settle: float, samples: int,
            harness_args: str | None = None) -> dict:
    """Power and clock samples of one operation (or one harness run) running back to back."""
    cmd = [HARNESS, *harness_args.split()] if harness_args else [BENCH, op, *map(str, shape), str(iters)]
    print("case", " ".join(cmd[1:]), flush=True)
    proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
    try:
        time.sleep(settle)
        watts, mhz = [], []
        for _ in range(samples):
            if proc.poll() is not None:
                break
            w, c = sample()
            if w is not None:
                watts.append(w)
            if c is not None:
                mhz.append(c)
        out, err = proc.communicate(timeout=600)
    finally:
        if proc.poll() is None:
            proc.kill()
            proc.wait()
    if proc.returncode != 0:
        raise RuntimeError(f"{op}: exit {proc.returncode}: {err.strip()[-400:]}")
    if not watts:
        raise RuntimeError(f"{op}: finished before a sample was taken; raise ITERS")
    result = parse_result(out.strip().splitlines()[-1])
    avg_us = result.get("avg_us")
    if harness_args:
        ms = result.get("gpu_ms_per_iter")
        avg_us = ms * 1e3 if isinstance(ms, float) else None
    rec = {"op": op, "iters": iters, "socket_w": statistics.median(watts), "sclk_mhz": statistics.median(mhz) if mhz else None,
           "samples": len(watts), "avg_us": avg_us}
    if rec["avg_us"] is not None:
        rec["energy_mj"] = rec["socket_w"] * rec["avg_us"] * 1e-3
    return rec


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("ops", nargs="*", help="OP:ITERS pairs")
    ap.add_argument("--harness", action="append", default=[], metavar="ARGS",
                    help="a llama2c_hip command line (its arguments) to sample as well")
    ap.add_argument("--shape", nargs=3, type=int, default=[1024, 16384, 8192], metavar=("BATCH", "SIZE", "ROWS"))
    ap.add_argument("--settle", type=float, default=2.0, help="seconds before the first sample")
    ap.add_argument("--samples", type=int, default=3)
    ap.add_argument("--idle-settle", type=float, default=8.0, help="seconds without work before the idle reading")
    ap.add_argument("--out")
    a = ap.parse_args(argv)
    time.sleep(a.idle_settle)
    idle, idle_clk = sample()
    print(f"idle socket_w={idle} sclk_mhz={idle_clk}", flush=True)
    recs = []
    for spec in a.ops:
        op, _, iters = spec.partition(":")
        rec = measure(op, int(iters or 1000), tuple(a.shape), a.settle, a.samples)
        if idle is not None and rec.get("avg_us") is not None:
            rec["energy_above_idle_mj"] = (rec["socket_w"] - idle) * rec["avg_us"] * 1e-3
        recs.append(rec)
        print(" ".join(f"{k}={v:.4g}" if isinstance(v, float) else f"{k}={v}" for k, v in rec.items()), flush=True)
    for args in a.harness:
        rec = measure("llama2c_hip " + args, 0, tuple(a.shape), a.settle, a.samples, harness_args=args)
        if idle is not None and rec.get("avg_us") is not None:
            rec["energy_above_idle_mj"] = (rec["socket_w"] - idle) * rec["avg_us"] * 1e-3
        recs.append(rec)
        print(" ".join(f"{k}={v:.4g}" if isinstance(v, float) else f"{k}={v}" for k, v in rec.items()), flush=True)
    if a.out:
        with open(a.out, "w") as f:
            json.dump({"idle_w": idle, "ops": recs}, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
