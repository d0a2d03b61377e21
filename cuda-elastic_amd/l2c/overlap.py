"""How other kernels overlap a product kernel in a rocprofv3 kernel trace.

For every launch of the product kernel (the kernel whose name contains the
given fragment), the row kernels that start in its window are attributed to
it. For each row kernel name the reducer reports, as medians over the
iterations in the middle half of the trace (the steady state):

- its start and end relative to the product's start (negative: it started
  first);
- the fraction of its duration spent inside the product's span;

and for the product, the median duration, the median gap from one launch's
end to the next launch's start, and the median iteration period (start to
start).

    python -m l2c.overlap DIR --product scaled_gemm_wide --rows rmsnorm softmax [--out FILE.json]

The figures show whether a three-stream iteration (llama2c_cuda_graph.cu:
347-381) runs its row kernels beside the product or after it.
"""
from __future__ import annotations

import argparse
import bisect
import csv
import glob
import json
import os
import statistics
import sys


def _find(directory: str, suffix: str) -> str | None:
    hits = sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))
    return hits[0] if hits else None


def summarize(kernel_rows: list[dict], product: str, rows: list[str]) -> dict:
    """Overlap figures of one kernel trace (timestamps in nanoseconds).

    A row kernel belongs to the product launch whose window it starts in: after
    the previous launch of the product ended and before this one ends. Only
    the product launches whose window holds a kernel of the first row fragment
    count as iterations (the harness also times the product alone, back to
    back), and the figures are medians over the middle half of those."""
    spans = sorted(((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]) for r in kernel_rows))
    prods = [s for s in spans if product in s[2]]
    if len(prods) < 2:
        raise ValueError(f"fewer than two launches of a kernel matching {product!r}")
    others = [s for s in spans if product not in s[2]]
    other_starts = [o[0] for o in others]
    windows = []
    for i, (ps, pe, _) in enumerate(prods):
        a = bisect.bisect_left(other_starts, prods[i - 1][1]) if i > 0 else 0
        windows.append(others[a:bisect.bisect_left(other_starts, pe)])
    marker = rows[0]
    its = [i for i in range(len(prods)) if any(marker in o[2] for o in windows[i])]
    if not its:
        raise ValueError(f"no launch of {product!r} has a {marker!r} kernel in its window")
    m = len(its)
    steady = its[m // 4: 3 * m // 4] if m >= 4 else its
    out: dict = {
        "product": prods[steady[0]][2][:80],
        "launches": len(prods),
        "iterations": m,
        "steady_iterations": len(steady),
        "product_us": round(statistics.median((prods[i][1] - prods[i][0]) / 1000.0 for i in steady), 3),
    }
    is_it = set(its)
    nxt = [i for i in steady if i + 1 in is_it]
    out["gap_us"] = round(statistics.median((prods[i + 1][0] - prods[i][1]) / 1000.0 for i in nxt), 3) if nxt else None
    out["period_us"] = round(statistics.median((prods[i + 1][0] - prods[i][0]) / 1000.0 for i in nxt), 3) if nxt else None
    out["rows"] = {}
    for frag in rows:
        rel_start, rel_end, inside = [], [], []
        for i in steady:
            ps, pe, _ = prods[i]
            for s, e, name in windows[i]:
                if frag not in name:
                    continue
                rel_start.append((s - ps) / 1000.0)
                rel_end.append((e - ps) / 1000.0)
                inside.append(max(0, min(e, pe) - max(s, ps)) / max(e - s, 1))
        if rel_start:
            out["rows"][frag] = {
                "n": len(rel_start),
                "start_us": round(statistics.median(rel_start), 3),
                "end_us": round(statistics.median(rel_end), 3),
                "inside_product": round(statistics.median(inside), 3),
            }
        else:
            out["rows"][frag] = {"n": 0}
    return out


def summarize_dir(directory: str, product: str, rows: list[str]) -> dict:
    path = _find(directory, "kernel_trace.csv")
    if not path:
        raise FileNotFoundError(f"no *kernel_trace.csv under {directory}")
    with open(path, newline="") as f:
        return summarize(list(csv.DictReader(f)), product, rows)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("directory")
    ap.add_argument("--product", required=True, help="fragment of the product kernel's name")
    ap.add_argument("--rows", nargs="+", default=["rmsnorm", "softmax"], help="fragments of the row kernels' names")
    ap.add_argument("--out", help="write the JSON summary here as well")
    a = ap.parse_args(argv)
    s = summarize_dir(a.directory, a.product, a.rows)
    text = json.dumps(s, indent=1)
    print(text)
    if a.out:
        with open(a.out, "w") as f:
            f.write(text + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
