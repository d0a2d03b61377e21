"""Harness-level checks of the drop-in command line, as run plans.

Two checks of the reference are restated here:

* the check matrix (llama2c/Makefile:24-28, 44-56): every combination of
  shape x input set x matmul variant x launch mode x copy mode must exit 0
  with valid=1;
* the dump comparison (llama2c/compare_sota.sh:41-71): on identical inputs,
  the graph and direct runs of the coalesced product, the fused single launch
  and the naive product each write an L2CDUMP file, and the dumps must agree
  within the oracle tolerances (bin/l2c_compare).

A plan is a list of Case records built up front, so tests can inspect it and
the command line can print it; execution goes through the same harness entry
point as the tests (l2c.harness, in this process) and the dump comparer.

    python -m l2c.matrix check   [--shapes B,S,R,REPEATS ...] [--inputs ...] [--variants ...]
    python -m l2c.matrix compare [--shapes B,S,R ...] [--inputs ...] [--copies nocopy copy] [--keep DIR]
"""
import argparse
import dataclasses
import os
import sys
import tempfile
import time
from typing import List, Optional, Sequence, Tuple

# The reference's shapes: the sheet shape, a size that is not a multiple of 4,
# and odd sizes with two repeats (llama2c/Makefile:44-56).
SHEET = (1024, 16384, 8192, 1)
CHECK_SHAPES = [(64, 1000, 300, 1), (33, 1001, 77, 2), SHEET]
CHECK_INPUTS = ["deterministic", "random=1", "random=2"]
CHECK_VARIANTS = ["coalesced", "naive", "fused", "batched"]
COMPARE_SHAPES = [(1024, 16384, 8192), (64, 1000, 300), (33, 1001, 77)]
COMPARE_INPUTS = ["deterministic", "random=1", "random=2", "random=3"]
# The four producers whose dumps must agree (compare_sota.sh:57-63 compares the
# graph, direct and SOTA binaries; the naive product is this build's fourth).
COMPARE_PRODUCERS = [("graph", "graph", "coalesced"), ("direct", "direct", "coalesced"),
                     ("fused", "graph", "fused"), ("naive", "direct", "naive")]


@dataclasses.dataclass(frozen=True)
class Case:
    label: str
    mode: str
    variant: str
    batch: int
    size: int
    rows: int
    repeats: int
    copies: str
    inputs: str
    launches: str = "auto"
    warmup_ms: int = 1

    def argv(self, dump: Optional[str] = None) -> List[str]:
        a = [self.mode, self.launches, self.batch, self.size, self.rows, self.repeats, self.warmup_ms,
             self.copies, self.variant, self.inputs]
        if dump:
            a.append(f"--dump={dump}")
        return [str(x) for x in a]


def check_plan(shapes: Sequence[Tuple[int, int, int, int]] = CHECK_SHAPES,
               inputs: Sequence[str] = CHECK_INPUTS,
               variants: Sequence[str] = CHECK_VARIANTS,
               modes: Sequence[str] = ("graph", "direct"),
               copies: Sequence[str] = ("nocopy", "copy")) -> List[Case]:
    return [Case(f"{v}/{m}/{c}", m, v, b, s, r, rep, c, i)
            for (b, s, r, rep) in shapes for i in inputs for v in variants for m in modes for c in copies]


def compare_plan(shapes: Sequence[Tuple[int, int, int]] = COMPARE_SHAPES,
                 inputs: Sequence[str] = COMPARE_INPUTS,
                 copies: Sequence[str] = ("nocopy",)) -> List[List[Case]]:
    """Groups of runs whose dumps must agree: one group per shape x copy mode
    x input set, one case per producer."""
    return [[Case(label, mode, variant, b, s, r, 1, c, i, launches="3")
             for (label, mode, variant) in COMPARE_PRODUCERS]
            for (b, s, r) in shapes for c in copies for i in inputs]


@dataclasses.dataclass
class Outcome:
    case: Case
    code: int
    record: dict
    raw: str
    seconds: float

    @property
    def ok(self) -> bool:
        return self.code == 0 and self.record.get("valid") == 1


def execute(case: Case, dump: Optional[str] = None) -> Outcome:
    import l2c
    t = time.time()
    code, rec, raw = l2c.harness(case.argv(dump))
    return Outcome(case, code, rec or {}, raw, time.time() - t)


def summary(o: Outcome) -> str:
    r = o.record
    us = r.get("gpu_ms_per_iter")
    us = f"{1000.0 * us:10.2f} us" if isinstance(us, (int, float)) else " " * 13
    return (f"{o.case.label:24s} {o.case.batch}x{o.case.size}x{o.case.rows} {o.case.inputs:13s} "
            f"{us} valid={r.get('valid', '?')} exit={o.code}")


def run_check(plan: List[Case], out=sys.stdout) -> int:
    failed = 0
    for case in plan:
        o = execute(case)
        print(summary(o), file=out, flush=True)
        if not o.ok:
            failed += 1
            print(o.raw, file=out)
    print(f"check: {len(plan) - failed} of {len(plan)} runs valid", file=out)
    return 1 if failed else 0


def compare_group(group: List[Case], directory: str, out=sys.stdout) -> bool:
    """Runs one group with dumps into `directory` and compares them; True when
    every run is valid and the comparer accepts the dumps."""
    import l2c
    dumps, ok = [], True
    for case in group:
        path = os.path.join(directory, f"{case.label}.bin")
        o = execute(case, dump=path)
        print("  " + summary(o), file=out, flush=True)
        if not o.ok:
            ok = False
            print(o.raw, file=out)
        dumps.append(path)
    if ok:
        code, text = l2c.compare_dumps(dumps)
        print(text.rstrip(), file=out)
        ok = code == 0
    for p in dumps:
        if os.path.exists(p):
            os.remove(p)
    return ok


def run_compare(groups: List[List[Case]], keep: Optional[str] = None, out=sys.stdout) -> int:
    failed = 0
    with tempfile.TemporaryDirectory(prefix="l2c-compare-") as tmp:
        directory = keep or tmp
        os.makedirs(directory, exist_ok=True)
        for group in groups:
            c = group[0]
            print(f"== {c.batch}x{c.size}x{c.rows} {c.copies} {c.inputs}", file=out, flush=True)
            if not compare_group(group, directory, out):
                failed += 1
    print(f"compare: {len(groups) - failed} of {len(groups)} configurations match", file=out)
    return 1 if failed else 0


def _shape(text: str) -> Tuple[int, ...]:
    return tuple(int(v) for v in text.split(","))


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m l2c.matrix")
    sub = ap.add_subparsers(dest="what", required=True)
    c = sub.add_parser("check", help="the reference's check matrix")
    c.add_argument("--shapes", nargs="+", type=_shape, default=CHECK_SHAPES, help="B,S,R,REPEATS")
    c.add_argument("--inputs", nargs="+", default=CHECK_INPUTS)
    c.add_argument("--variants", nargs="+", default=CHECK_VARIANTS)
    m = sub.add_parser("compare", help="graph / direct / fused / naive dumps must agree")
    m.add_argument("--shapes", nargs="+", type=_shape, default=COMPARE_SHAPES, help="B,S,R")
    m.add_argument("--inputs", nargs="+", default=COMPARE_INPUTS)
    m.add_argument("--copies", nargs="+", default=["nocopy"])
    m.add_argument("--keep", help="write the dumps here instead of a temporary directory")
    args = ap.parse_args(argv)
    import l2c
    l2c.load_host()
    if args.what == "check":
        return run_check(check_plan(args.shapes, args.inputs, args.variants))
    return run_compare(compare_plan(args.shapes, args.inputs, args.copies), keep=args.keep)


if __name__ == "__main__":
    sys.exit(main())
