#!/usr/bin/env python3
"""Compare two backends (or two runs) over gg_bench result CSVs.

The accounting of the reference's scripts/compare.py:1-28 (cases where both pass, wins,
geomean speedup, total time, mean TFLOPS, worst cases), written for this driver's CSV schema
(bench/bench_main.cpp:316-381 columns, as gg_bench writes them).

  compare.py RESULTS...                         mi355x vs hipblaslt_loop in the given CSVs/dirs
  compare.py --ours mi355x --other hipblaslt_grouped RESULTS...
  compare.py --base OLD.csv --new NEW.csv       one backend, two runs (e.g. before/after a change)
"""
from __future__ import annotations

import argparse
import csv
import glob
import math
import os
import sys
from typing import Dict, List, Tuple

OK = ("PASS", "SKIP")  # SKIP: timed with --no-check


def read_rows(paths: List[str]) -> List[dict]:
    files: List[str] = []
    for p in paths:
        files += sorted(glob.glob(os.path.join(p, "*.csv"))) if os.path.isdir(p) else [p]
    rows: List[dict] = []
    for f in files:
        with open(f, newline="") as fh:
            rows += list(csv.DictReader(fh))
    return rows


def index(rows: List[dict], key_fn) -> Dict[Tuple, Dict[str, dict]]:
    by: Dict[Tuple, Dict[str, dict]] = {}
    for r in rows:
        by.setdefault((int(r["TestID"]), r.get("Dtype", "")), {})[key_fn(r)] = r
    return by


def summarize(pairs, name_a: str, name_b: str, failed, worst: int = 8) -> List[str]:
    """pairs: [(key, row_a, row_b)] where both passed. a is the side whose wins are counted."""
    out: List[str] = []
    n = len(pairs)
    if n == 0:
        return [f"no case where both {name_a} and {name_b} passed"]
    wins = sum(float(a["TFLOPS"]) > float(b["TFLOPS"]) for _, a, b in pairs)
    geo = math.exp(sum(math.log(float(b["Time_ms"]) / float(a["Time_ms"])) for _, a, b in pairs) / n)
    ta = sum(float(a["Time_ms"]) for _, a, _ in pairs)
    tb = sum(float(b["Time_ms"]) for _, _, b in pairs)
    ma = sum(float(a["TFLOPS"]) for _, a, _ in pairs) / n
    mb = sum(float(b["TFLOPS"]) for _, _, b in pairs) / n
    out.append(f"{n} cases where both pass; {name_a} faster in {wins}/{n}; "
               f"cases with a non-passing side: {sorted(k[0] for k in failed)[:10]}")
    out.append(f"geomean speedup {name_a} vs {name_b}: {geo:.3f}x; total time {ta:.3f} ms vs {tb:.3f} ms "
               f"({tb / ta:.3f}x)")
    out.append(f"mean TFLOPS: {name_a} {ma:.1f}  {name_b} {mb:.1f}")
    out.append(f"worst cases for {name_a} ({name_a}/{name_b} TFLOPS):")
    for key, a, b in sorted(pairs, key=lambda t: float(t[1]["TFLOPS"]) / float(t[2]["TFLOPS"]))[:worst]:
        out.append(f"  {key[0]:4d} {a['Case'][:28]:28s} B={a['B']:>3} M={a['M']:>5} N={a['N']:>5} "
                   f"K={a['K']:>5}  {float(a['TFLOPS']):7.1f} vs {float(b['TFLOPS']):7.1f}  "
                   f"({float(a['TFLOPS']) / float(b['TFLOPS']):.2f})")
    return out


def compare_backends(rows: List[dict], ours: str, other: str) -> List[str]:
    by = index(rows, lambda r: r["Backend"])
    pairs, failed = [], []
    for key, d in sorted(by.items()):
        if ours in d and other in d:
            if d[ours]["Check"] == "PASS" and d[other]["Check"] in OK:
                pairs.append((key, d[ours], d[other]))
            elif d[ours]["Check"] not in OK or d[other]["Check"] not in OK + ("N/A",):
                failed.append(key)
    return summarize(pairs, ours, other, failed)


def compare_runs(base: List[dict], new: List[dict], backend: str) -> List[str]:
    b = {k: v[backend] for k, v in index(base, lambda r: r["Backend"]).items() if backend in v}
    n = {k: v[backend] for k, v in index(new, lambda r: r["Backend"]).items() if backend in v}
    pairs = [(k, n[k], b[k]) for k in sorted(set(b) & set(n))
             if n[k]["Check"] in OK and b[k]["Check"] in OK]
    failed = [k for k in sorted(set(b) & set(n)) if n[k]["Check"] not in OK or b[k]["Check"] not in OK]
    return summarize(pairs, f"new {backend}", f"base {backend}", failed)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("results", nargs="*", help="gg_bench CSVs or directories of them")
    ap.add_argument("--ours", default="mi355x")
    ap.add_argument("--other", default="hipblaslt_loop")
    ap.add_argument("--base", nargs="+", help="baseline run CSVs (with --new)")
    ap.add_argument("--new", nargs="+", help="new run CSVs (with --base)")
    a = ap.parse_args(argv)
    if a.base or a.new:
        if not (a.base and a.new):
            ap.error("--base and --new go together")
        lines = compare_runs(read_rows(a.base), read_rows(a.new), a.ours)
    else:
        if not a.results:
            ap.error("no result CSVs given")
        lines = compare_backends(read_rows(a.results), a.ours, a.other)
    print("\n".join(lines))
    return 0


if __name__ == "__main__":
    sys.exit(main())
