"""Graph-vs-direct sweeps of the llama2c harness and their speedup summary.

The experiment definitions follow llama2c/profile_cuda.sh:67-126 of the
reference (the `sweep` and `sweep-fill` config sets, trials with alternating
launch-mode order, the per-run CSV columns) and the derived metrics of
llama2c/plot_sweep.py:29-73 (per-trial direct/graph ratios of GPU time and host
submission time, graph setup cost, break-even replay count), so CSVs from
either side line up column for column. Plotting is not reproduced.

    python -m l2c.sweep sweep       [--out DIR] [--trials N] [--configs ...]
    python -m l2c.sweep sweep-fill  [--out DIR]
    python -m l2c.sweep speedup SWEEP.csv    (writes SWEEP-speedup.csv)

A config is batch,size,rows[,repeats[,copy|nocopy]] (repeats default 1,
copies default copy).
"""
from __future__ import annotations

import argparse
import csv
import math
import os
import subprocess
import sys
import time
from collections import OrderedDict

from . import HARNESS, parse_line

# The reference's experiment sets (profile_cuda.sh:107-124).
SWEEP_CONFIGS = ("1,16,16,1,nocopy 1,64,64,1,nocopy 1,64,64,16,nocopy 1,256,256,1,copy "
                 "1,256,256,8,nocopy 1,256,256,32,nocopy 1,1024,1024,1,nocopy 1,4096,4096,1,copy "
                 "512,16384,8192,1,copy")
SWEEP_LAUNCHES, SWEEP_MATMUL = "30", "naive"
FILL_CONFIGS = ("1024,256,8192,1,nocopy 1024,256,8192,8,nocopy 1024,256,8192,32,nocopy "
                "1024,1024,8192,1,nocopy 1024,1024,8192,8,nocopy 1024,1024,8192,32,nocopy "
                "1024,4096,8192,1,nocopy 1024,4096,8192,8,nocopy "
                "1024,16384,8192,1,nocopy 1024,16384,8192,8,nocopy")
FILL_LAUNCHES, FILL_MATMUL = "auto", "coalesced"

RESULT_FIELDS = ("gpu_ms_per_iter", "wall_ms_per_iter", "submit_us_per_iter", "graph_capture_ms",
                 "graph_instantiate_ms", "graph_upload_ms", "rms_waves", "softmax_waves",
                 "matmul_waves", "min_waves", "achieved_gbps", "valid")
HEADER = ("trial", "mode", "launches", "batch", "size", "rows", "repeats", "copies", "matmul",
          "warmup_ms") + RESULT_FIELDS + ("exit_code",)


def parse_config(text: str):
    parts = text.split(",")
    if not 3 <= len(parts) <= 5:
        raise ValueError(f"config {text!r}: expected batch,size,rows[,repeats[,copy|nocopy]]")
    batch, size, rows = (int(p) for p in parts[:3])
    repeats = int(parts[3]) if len(parts) > 3 and parts[3] else 1
    copies = parts[4] if len(parts) > 4 and parts[4] else "copy"
    if copies not in ("copy", "nocopy"):
        raise ValueError(f"config {text!r}: copies must be copy or nocopy")
    return batch, size, rows, repeats, copies


def run_sweep(name, configs, launches, matmul, trials=3, warmup_ms=100, out_dir=".",
              harness=HARNESS, stamp=None, timeout=600, log=print):
    """Runs every config `trials` times in both launch modes (direct first on
    odd trials, graph first on even ones) and writes one CSV row per run.
    Returns the CSV path."""
    os.makedirs(out_dir, exist_ok=True)
    stamp = stamp or time.strftime("%Y%m%d-%H%M%S")
    path = os.path.join(out_dir, f"{name}-{stamp}.csv")
    with open(path, "w", newline="") as stream:
        out = csv.writer(stream)
        out.writerow(HEADER)
        for config in configs.split():
            batch, size, rows, repeats, copies = parse_config(config)
            for trial in range(1, trials + 1):
                for mode in (("direct", "graph") if trial % 2 else ("graph", "direct")):
                    args = [mode, launches, batch, size, rows, repeats, warmup_ms, copies, matmul]
                    proc = subprocess.run([harness] + [str(a) for a in args], capture_output=True,
                                          text=True, timeout=timeout)
                    lines = proc.stdout.strip().splitlines()
                    fields = parse_line(lines[-1]) if proc.returncode == 0 and lines else {}
                    if proc.returncode == 0 and fields:
                        row = [trial, mode, fields.get("launches", launches), batch, size, rows,
                               repeats, copies, matmul, warmup_ms]
                        row += [fields.get(k, "") for k in RESULT_FIELDS]
                    else:
                        # A failed run keeps its identity; valid is 0.
                        row = [trial, mode, launches, batch, size, rows, repeats, copies, matmul,
                               warmup_ms] + [""] * (len(RESULT_FIELDS) - 1) + [0]
                        log(f"warning: {mode} failed for {config}: {proc.stderr.strip()[-300:]}")
                    out.writerow(row + [proc.returncode])
                    stream.flush()
                    log(f"[sweep] {name} {config} trial {trial} {mode}: exit {proc.returncode} "
                        f"gpu_ms_per_iter={fields.get('gpu_ms_per_iter')}")
    return path


def _mean(values):
    return sum(values) / len(values) if values else float("nan")


def speedup_rows(path):
    """Pairs direct and graph runs of each valid config by trial and derives
    the speedups (plot_sweep.py:29-73); configs keep sweep order."""
    groups: "OrderedDict[tuple, OrderedDict[str, dict]]" = OrderedDict()
    with open(path, newline="") as stream:
        for row in csv.DictReader(stream):
            if row.get("valid") != "1" or row.get("exit_code") != "0":
                continue
            key = (row["batch"], row["size"], row["rows"], row["repeats"], row["copies"],
                   row.get("matmul") or "naive")
            groups.setdefault(key, OrderedDict()).setdefault(row["trial"], {})[row["mode"]] = row
    results = []
    for key, trials in groups.items():
        pairs = [t for t in trials.values() if "direct" in t and "graph" in t]
        if not pairs:
            continue

        def col(mode, field):
            return [float(t[mode][field]) for t in pairs]

        def opt(mode, field):
            vals = [float(t[mode][field]) for t in pairs if t[mode].get(field)]
            return _mean(vals) if vals else ""

        def ratio(field):
            return [d / g for d, g in zip(col("direct", field), col("graph", field))]

        gpu, submit = ratio("gpu_ms_per_iter"), ratio("submit_us_per_iter")
        setup = _mean([sum(float(t["graph"][f]) for f in
                           ("graph_capture_ms", "graph_instantiate_ms", "graph_upload_ms")) for t in pairs])
        saving = _mean(col("direct", "wall_ms_per_iter")) - _mean(col("graph", "wall_ms_per_iter"))
        results.append(OrderedDict([
            ("batch", int(key[0])), ("size", int(key[1])), ("rows", int(key[2])),
            ("repeats", int(key[3])), ("copies", key[4]), ("matmul", key[5]), ("trials", len(pairs)),
            ("min_waves", opt("direct", "min_waves")),
            ("direct_gbps", opt("direct", "achieved_gbps")), ("graph_gbps", opt("graph", "achieved_gbps")),
            ("direct_gpu_ms", _mean(col("direct", "gpu_ms_per_iter"))),
            ("graph_gpu_ms", _mean(col("graph", "gpu_ms_per_iter"))),
            ("gpu_speedup", _mean(gpu)), ("gpu_speedup_min", min(gpu)), ("gpu_speedup_max", max(gpu)),
            ("direct_submit_us", _mean(col("direct", "submit_us_per_iter"))),
            ("graph_submit_us", _mean(col("graph", "submit_us_per_iter"))),
            ("submit_speedup", _mean(submit)), ("submit_speedup_min", min(submit)),
            ("submit_speedup_max", max(submit)),
            ("graph_setup_ms", setup),
            ("break_even_replays", math.ceil(setup / saving) if saving > 0 else ""),
        ]))
    return results


def write_speedup(path):
    rows = speedup_rows(path)
    out_path = path[:-4] + "-speedup.csv" if path.endswith(".csv") else path + "-speedup.csv"
    with open(out_path, "w", newline="") as stream:
        if rows:
            w = csv.DictWriter(stream, fieldnames=list(rows[0].keys()))
            w.writeheader()
            w.writerows(rows)
    return out_path, rows


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m l2c.sweep", description=__doc__.split("\n\n")[0])
    ap.add_argument("action", choices=("sweep", "sweep-fill", "speedup"))
    ap.add_argument("csv", nargs="?", help="sweep CSV (speedup)")
    ap.add_argument("--out", default="profiles-sweep", help="output directory")
    ap.add_argument("--configs", default=None)
    ap.add_argument("--launches", default=None)
    ap.add_argument("--matmul", default=None)
    ap.add_argument("--trials", type=int, default=3)
    ap.add_argument("--warmup-ms", type=int, default=100)
    a = ap.parse_args(argv)
    if a.action == "speedup":
        if not a.csv:
            ap.error("speedup needs the sweep CSV")
        out, rows = write_speedup(a.csv)
        print(f"{len(rows)} configs -> {out}")
        return 0
    configs, launches, matmul = ((SWEEP_CONFIGS, SWEEP_LAUNCHES, SWEEP_MATMUL) if a.action == "sweep"
                                 else (FILL_CONFIGS, FILL_LAUNCHES, FILL_MATMUL))
    path = run_sweep(a.action, a.configs or configs, a.launches or launches, a.matmul or matmul,
                     trials=a.trials, warmup_ms=a.warmup_ms, out_dir=a.out,
                     log=lambda *m: print(*m, file=sys.stderr, flush=True))
    out, rows = write_speedup(path)
    print(f"Sweep results: {path}\nSpeedup summary: {out} ({len(rows)} configs)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
