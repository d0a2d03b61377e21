"""Per-kernel averages of a rocprofv3 counter collection.

Reads the `*counter_collection.csv` that `rocprofv3 --pmc ... --output-format
csv -d DIR` writes and prints, for every kernel whose name contains the
filter, each counter's mean value per dispatch (counters with several
instances are summed over them by rocprofv3 first), the number of dispatches,
and the mean dispatch duration when the trace has one. Derived figures the
counter pages quote are computed from these means:

    busy       SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE * CUs)
    clock GHz  GRBM_GUI_ACTIVE / dispatch duration

    python -m l2c.pmc DIR [--kernel SUBSTRING] [--skip N] [--json]

--skip drops each kernel's first N dispatches (warm-up launches at a lower
clock).
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
import sys


def load(directory: str) -> list[dict]:
    paths = sorted(glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True))
    if not paths:
        raise FileNotFoundError(f"no *counter_collection.csv under {directory}")
    rows: list[dict] = []
    for p in paths:
        rows.extend(csv.DictReader(open(p)))
    return rows


def per_kernel(rows: list[dict], kernel_filter: str = "", skip: int = 0) -> dict:
    """{kernel: {"dispatches": n, "counters": {name: mean}, "duration_us": mean or None}}."""
    values: dict[str, dict[str, dict[str, float]]] = {}
    durations: dict[str, dict[str, float]] = {}
    for r in rows:
        name = r.get("Kernel_Name", "")
        if kernel_filter and kernel_filter not in name:
            continue
        dispatch = r.get("Dispatch_Id", "")
        counter = r.get("Counter_Name", "")
        v = float(r.get("Counter_Value", "nan"))
        per = values.setdefault(name, {}).setdefault(dispatch, {})
        per[counter] = per.get(counter, 0.0) + v
        if r.get("Start_Timestamp") and r.get("End_Timestamp"):
            durations.setdefault(name, {})[dispatch] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
    out = {}
    for name, by_dispatch in values.items():
        ids = sorted(by_dispatch, key=lambda d: int(d) if d.isdigit() else d)[skip:]
        if not ids:
            continue
        counters = sorted({c for d in ids for c in by_dispatch[d]})
        means = {c: statistics.mean(by_dispatch[d].get(c, 0.0) for d in ids) for c in counters}
        dur = [durations.get(name, {}).get(d) for d in ids]
        dur = [x for x in dur if x is not None]
        out[name] = {"dispatches": len(ids), "counters": means,
                     "duration_us": statistics.mean(dur) if dur else None}
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("directory")
    ap.add_argument("--kernel", default="")
    ap.add_argument("--skip", type=int, default=0)
    ap.add_argument("--json", action="store_true")
    a = ap.parse_args(argv)
    result = per_kernel(load(a.directory), a.kernel, a.skip)
    if a.json:
        print(json.dumps(result))
        return 0
    for name, k in result.items():
        dur = f", {k['duration_us']:.2f} us" if k["duration_us"] is not None else ""
        print(f"{name[:100]}  ({k['dispatches']} dispatches{dur})")
        for c, v in k["counters"].items():
            print(f"    {c:40s} {v:18.1f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
