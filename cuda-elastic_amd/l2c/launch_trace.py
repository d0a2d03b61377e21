"""Launch-cost summary of a rocprofv3 HIP API + kernel trace.

Reduces the `*hip_api_trace.csv` and `*kernel_trace.csv` that
`rocprofv3 --hip-trace --kernel-trace --output-format csv -d DIR` writes to
the figures that locate where a replayed iteration's time goes:

- per HIP API function: calls, mean and median duration (host time in the
  runtime);
- per kernel: launches and mean duration (device time);
- the steady state (the middle half of the kernels by start time): the span
  it covers, the kernels' busy time in it, and the idle gap between one
  kernel's end and the next one's start;
- per launching API function: the median time from the call's return to the
  start of the kernel it submitted (negative when the kernel starts before
  the call returns).

    python -m l2c.launch_trace DIR [--out FILE.json]

The trace is the sweep tooling's companion for the graph-against-direct
question of llama2c/profile_cuda.sh:67-126 (the reference answers it with
nsys timelines); only the reduced JSON needs keeping.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
import sys


def _find(directory: str, suffix: str) -> str | None:
    hits = sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))
    return hits[0] if hits else None


def _us(row: dict, start: str = "Start_Timestamp", end: str = "End_Timestamp") -> float:
    return (int(row[end]) - int(row[start])) / 1000.0


def summarize(api_rows: list[dict], kernel_rows: list[dict], top: int = 12) -> dict:
    """The launch-cost figures of one trace (timestamps in nanoseconds)."""
    by_function: dict[str, list[float]] = {}
    for r in api_rows:
        by_function.setdefault(r["Function"], []).append(_us(r))
    ranked = sorted(by_function.items(), key=lambda kv: -sum(kv[1]))[:top]
    out: dict = {"api": {f: {"n": len(v), "mean_us": round(statistics.mean(v), 3),
                             "median_us": round(statistics.median(v), 3)} for f, v in ranked}}
    by_kernel: dict[str, list[dict]] = {}
    for r in kernel_rows:
        by_kernel.setdefault(r["Kernel_Name"][:60], []).append(r)
    out["kernels"] = {k: {"n": len(v), "mean_us": round(statistics.mean(_us(x) for x in v), 3)}
                      for k, v in by_kernel.items()}
    ordered = sorted(kernel_rows, key=lambda r: int(r["Start_Timestamp"]))
    n = len(ordered)
    middle = ordered[n // 4: 3 * n // 4]
    if len(middle) >= 2:
        span = (int(middle[-1]["End_Timestamp"]) - int(middle[0]["Start_Timestamp"])) / 1000.0
        busy = sum(_us(r) for r in middle)
        gaps = [(int(b["Start_Timestamp"]) - int(a["End_Timestamp"])) / 1000.0 for a, b in zip(middle, middle[1:])]
        out["steady"] = {"kernels": len(middle), "span_us": round(span, 1), "kernel_busy_us": round(busy, 1),
                         "busy_frac": round(busy / span, 3) if span > 0 else None,
                         "gap_median_us": round(statistics.median(gaps), 3),
                         "gap_mean_us": round(statistics.mean(gaps), 3)}
    start_by_correlation = {r.get("Correlation_Id"): int(r["Start_Timestamp"]) for r in kernel_rows}
    latency: dict[str, list[float]] = {}
    for r in api_rows:
        c = r.get("Correlation_Id")
        if c in start_by_correlation:
            latency.setdefault(r["Function"], []).append((start_by_correlation[c] - int(r["End_Timestamp"])) / 1000.0)
    out["call_end_to_kernel_start_us"] = {f: {"n": len(v), "median": round(statistics.median(v), 2)}
                                          for f, v in latency.items()}
    return out


def summarize_dir(directory: str) -> dict:
    api = _find(directory, "hip_api_trace.csv")
    kernels = _find(directory, "kernel_trace.csv")
    if kernels is None:
        raise FileNotFoundError(f"no *kernel_trace.csv under {directory}")
    api_rows = list(csv.DictReader(open(api))) if api else []
    return summarize(api_rows, list(csv.DictReader(open(kernels))))


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("directory")
    ap.add_argument("--out")
    a = ap.parse_args(argv)
    text = json.dumps(summarize_dir(a.directory))
    if a.out:
        with open(a.out, "w") as f:
            f.write(text + "\n")
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
