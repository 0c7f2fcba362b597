"""Summaries of rocprofv3 output for this library's kernels.

    python -m trispconv_amd.profiling trace  <out_dir>            # kernel-trace stats
    python -m trispconv_amd.profiling pmc    <out_dir> [--kernel SUBSTR]
    python -m trispconv_amd.profiling calib  <out_dir> --bytes N  [--kernel SUBSTR]

``out_dir`` is a rocprofv3 ``-d`` directory written with ``--output-format
csv``.  ``trace`` prints per-kernel call count and average / min / max /
total duration; ``pmc`` prints the per-dispatch average of every collected
counter for the kernels whose name contains SUBSTR; ``calib`` prints the
counter value per byte for a copy kernel of known size (the FETCH_SIZE /
WRITE_SIZE scale factor).
"""
from __future__ import annotations

import argparse
import csv
import sys
from collections import defaultdict
from pathlib import Path


def _rows(out_dir: Path, suffix: str):
    files = sorted(out_dir.rglob(f"*{suffix}"))
    if not files:
        raise SystemExit(f"no *{suffix} under {out_dir}")
    for f in files:
        with open(f, newline="") as fh:
            yield from csv.DictReader(fh)


def _short(name: str, width: int = 90) -> str:
    return name if len(name) <= width else name[: width - 3] + "..."


def trace(out_dir: Path) -> None:
    per = defaultdict(list)
    for r in _rows(out_dir, "kernel_trace.csv"):
        per[r["Kernel_Name"]].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in per.values())
    print(f"{'calls':>6} {'avg_us':>10} {'min_us':>10} {'max_us':>10} {'total_ms':>9} {'%':>6}  kernel")
    for name, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        print(f"{len(v):6d} {sum(v) / len(v):10.2f} {min(v):10.2f} {max(v):10.2f} "
              f"{sum(v) / 1e3:9.3f} {100 * sum(v) / total:6.2f}  {_short(name)}")


def _pmc(out_dir: Path, kernel: str):
    per = defaultdict(lambda: defaultdict(list))
    for r in _rows(out_dir, "counter_collection.csv"):
        if kernel and kernel not in r["Kernel_Name"]:
            continue
        key = (r["Kernel_Name"], r.get("Dispatch_Id", ""))
        per[r["Counter_Name"]][key].append(float(r["Counter_Value"]))
    out = {}
    for counter, dispatches in per.items():
        vals = [sum(v) for v in dispatches.values()]  # sum over dimensions of a dispatch
        out[counter] = (sum(vals) / len(vals), len(vals))
    return out


def pmc(out_dir: Path, kernel: str) -> None:
    for counter, (avg, n) in sorted(_pmc(out_dir, kernel).items()):
        print(f"{counter:34s} {avg:18.1f}  (avg over {n} dispatches)")


def calib(out_dir: Path, kernel: str, nbytes: int) -> None:
    for counter, (avg, n) in sorted(_pmc(out_dir, kernel).items()):
        print(f"{counter:34s} {avg:18.1f}  -> {avg / nbytes:.6f} per byte of a {nbytes}-byte copy"
              f" ({n} dispatches)")


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["trace", "pmc", "calib"])
    ap.add_argument("out_dir", type=Path)
    ap.add_argument("--kernel", default="")
    ap.add_argument("--bytes", type=int, default=0)
    a = ap.parse_args(argv)
    if a.mode == "trace":
        trace(a.out_dir)
    elif a.mode == "pmc":
        pmc(a.out_dir, a.kernel)
    else:
        calib(a.out_dir, a.kernel, a.bytes)


if __name__ == "__main__":
    main(sys.argv[1:])
