"""Summaries of rocprofv3 output for this library's kernels.

    python -m trispconv_amd.profiling trace  <out_dir>            # kernel-trace stats
    python -m trispconv_amd.profiling pmc    <out_dir> [--kernel SUBSTR] [--trace DIR --near-us T]
    python -m trispconv_amd.profiling calib  <out_dir> --bytes N  [--kernel SUBSTR]
    python -m trispconv_amd.profiling traffic --fetch DIR --write DIR --trace DIR
            --kernel SUBSTR --calib-kernel SUBSTR --calib-bytes N [--algorithmic-bytes B]
            [--near-us T]
    python -m trispconv_amd.profiling table --fetch DIR --write DIR --trace DIR
            --kernels SUB1,SUB2,... --calib-kernel SUBSTR --calib-bytes N [--algorithmic-bytes B]

``out_dir`` is a rocprofv3 ``-d`` directory written with ``--output-format
csv``.  ``trace`` prints per-kernel call count and average / min / max /
total duration; ``pmc`` prints the per-dispatch average of every collected
counter for the kernels whose name contains SUBSTR; ``calib`` prints the
counter value per byte for a copy kernel of known size (the FETCH_SIZE /
WRITE_SIZE scale factor); ``traffic`` combines a FETCH_SIZE pass, a WRITE_SIZE
pass (each holding one copy-like kernel that reads and writes N bytes) and a
kernel trace into HBM bytes per launch of one kernel, scaled by what the
counters read for the copy; ``table`` does the same for each kernel of a
multi-kernel step (the pair build) and adds up the step.

``--near-us T`` picks, among the kernel's dispatches grouped by grid size,
the group whose median duration is nearest T microseconds (one layer of a
network whose layers share a kernel template), and reports medians over that
group, so the few first-use dispatches of a layer (run before its execution
order exists) do not bias the figures.
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


def _grid(r) -> int:
    """Total work-items of a dispatch (counter rows carry Grid_Size, trace rows
    Grid_Size_X/Y/Z)."""
    if r.get("Grid_Size"):
        return int(r["Grid_Size"])
    return int(r.get("Grid_Size_X") or 1) * int(r.get("Grid_Size_Y") or 1) * \
        int(r.get("Grid_Size_Z") or 1)


def _median(v):
    v = sorted(v)
    n = len(v)
    return v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])


def _pmc(out_dir: Path, kernel: str, group=None, median: bool = False):
    per = defaultdict(lambda: defaultdict(list))
    for r in _rows(out_dir, "counter_collection.csv"):
        if kernel and kernel not in r["Kernel_Name"]:
            continue
        if group and (r["Kernel_Name"], _grid(r)) != group:
            continue
        key = (r["Kernel_Name"], r.get("Dispatch_Id", ""))
        per[r["Counter_Name"]][key].append(float(r["Counter_Value"]))
    out = {}
    for counter, dispatches in per.items():
        vals = [sum(v) for v in dispatches.values()]  # sum over dimensions of a dispatch
        out[counter] = (_median(vals) if median else sum(vals) / len(vals), len(vals))
    return out


def _grid_groups(trace_dir: Path, kernel: str):
    """Durations of the kernel's dispatches by (full kernel name, grid size)."""
    groups = defaultdict(list)
    for r in _rows(trace_dir, "kernel_trace.csv"):
        if kernel in r["Kernel_Name"]:
            groups[(r["Kernel_Name"], _grid(r))].append(
                (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return groups


def _pick_group(trace_dir: Path, kernel: str, near_us: float):
    """(name, grid size) of the dispatch group whose median duration is nearest near_us."""
    groups = _grid_groups(trace_dir, kernel)
    if not groups:
        raise SystemExit(f"no dispatches of {kernel} in {trace_dir}")
    return min(groups, key=lambda g: abs(_median(groups[g]) - near_us))


def pmc(out_dir: Path, kernel: str, trace_dir: Path = None, near_us: float = 0.0) -> None:
    group = _pick_group(trace_dir, kernel, near_us) if near_us and trace_dir else None
    if group:
        print(f"kernel_name: {_short(group[0], 120)}")
        print(f"grid_size: {group[1]}   (dispatch group nearest {near_us:.1f} us)")
    stat = "median" if group else "avg"
    for counter, (avg, n) in sorted(_pmc(out_dir, kernel, group, bool(group)).items()):
        print(f"{counter:34s} {avg:18.1f}  ({stat} over {n} dispatches)")


def calib(out_dir: Path, kernel: str, nbytes: int) -> None:
    for counter, (avg, n) in sorted(_pmc(out_dir, kernel).items()):
        print(f"{counter:34s} {avg:18.1f}  -> {avg / nbytes:.6f} per byte of a {nbytes}-byte copy"
              f" ({n} dispatches)")


def _avg_duration_us(trace_dir: Path, kernel: str):
    durs = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            for r in _rows(trace_dir, "kernel_trace.csv") if kernel in r["Kernel_Name"]]
    return (sum(durs) / len(durs), len(durs)) if durs else (float("nan"), 0)


def traffic(fetch_dir: Path, write_dir: Path, trace_dir: Path, kernel: str, calib_kernel: str,
            calib_bytes: int, algorithmic: float, near_us: float = 0.0) -> None:
    """FETCH_SIZE and WRITE_SIZE are in KiB per dispatch; each is divided by
    what it reads per byte of the copy-like calibration kernel."""
    group = _pick_group(trace_dir, kernel, near_us) if near_us else None
    med = bool(near_us)
    f_k, nf = _pmc(fetch_dir, kernel, group, med)["FETCH_SIZE"]
    w_k, nw = _pmc(write_dir, kernel, group, med)["WRITE_SIZE"]
    f_c, _ = _pmc(fetch_dir, calib_kernel)["FETCH_SIZE"]
    w_c, _ = _pmc(write_dir, calib_kernel)["WRITE_SIZE"]
    f_scale = f_c * 1024.0 / calib_bytes
    w_scale = w_c * 1024.0 / calib_bytes
    fetch_b = f_k * 1024.0 / f_scale
    write_b = w_k * 1024.0 / w_scale
    if group:
        durs = _grid_groups(trace_dir, kernel)[group]
        avg_us, nt = _median(durs), len(durs)
    else:
        avg_us, nt = _avg_duration_us(trace_dir, kernel)
    stat = "median" if med else "avg"
    print(f"kernel: {kernel}")
    if group:
        print(f"kernel_name: {_short(group[0], 120)}")
        print(f"grid_size: {group[1]}   (dispatch group nearest {near_us:.1f} us)")
    print(f"kernel_avg_us: {avg_us:.2f}   ({stat} over the dispatches)")
    print(f"kernel_trace_dispatches: {nt}")
    print(f"fetch_kib_per_dispatch: {f_k:.1f}   ({stat} over {nf} dispatches)")
    print(f"write_kib_per_dispatch: {w_k:.1f}   ({stat} over {nw} dispatches)")
    print(f"calib_fetch_counter_per_byte: {f_scale:.4f}   ({calib_kernel}, {calib_bytes} bytes)")
    print(f"calib_write_counter_per_byte: {w_scale:.4f}")
    print(f"fetch_bytes_per_launch: {fetch_b:.0f}")
    print(f"write_bytes_per_launch: {write_b:.0f}")
    print(f"traffic_bytes_per_launch: {fetch_b + write_b:.0f}")
    if algorithmic:
        print(f"algorithmic_bytes_per_launch: {algorithmic:.0f}")
        print(f"traffic_over_algorithmic: {(fetch_b + write_b) / algorithmic:.3f}")
    if avg_us == avg_us and avg_us > 0:
        print(f"hbm_gbs_at_avg_duration: {(fetch_b + write_b) / (avg_us * 1e3):.1f}")


def _scales(fetch_dir: Path, write_dir: Path, calib_kernel: str, calib_bytes: int):
    f_c, _ = _pmc(fetch_dir, calib_kernel)["FETCH_SIZE"]
    w_c, _ = _pmc(write_dir, calib_kernel)["WRITE_SIZE"]
    return f_c * 1024.0 / calib_bytes, w_c * 1024.0 / calib_bytes


def table(fetch_dir: Path, write_dir: Path, trace_dir: Path, kernels, calib_kernel: str,
          calib_bytes: int, algorithmic: float) -> None:
    """Per-kernel HBM bytes and rate for the kernels of one step, and the step's
    totals (kernel time only: launch gaps are not in the sum)."""
    f_scale, w_scale = _scales(fetch_dir, write_dir, calib_kernel, calib_bytes)
    print(f"calib: FETCH_SIZE {f_scale:.4f}, WRITE_SIZE {w_scale:.4f} counter KiB per KiB moved "
          f"({calib_kernel}, {calib_bytes} bytes)")
    print(f"{'kernel':28s} {'avg_us':>8} {'fetch_MB':>9} {'write_MB':>9} {'GB/s':>8}")
    tot_us = tot_b = 0.0
    for k in kernels:
        f_k = _pmc(fetch_dir, k).get("FETCH_SIZE", (0.0, 0))[0]
        w_k = _pmc(write_dir, k).get("WRITE_SIZE", (0.0, 0))[0]
        fb, wb = f_k * 1024.0 / f_scale, w_k * 1024.0 / w_scale
        us, _ = _avg_duration_us(trace_dir, k)
        tot_us += us
        tot_b += fb + wb
        print(f"{k:28s} {us:8.2f} {fb / 1e6:9.2f} {wb / 1e6:9.2f} {(fb + wb) / (us * 1e3):8.1f}")
    print(f"{'step (kernels only)':28s} {tot_us:8.2f} {tot_b / 1e6:19.2f} {tot_b / (tot_us * 1e3):8.1f}")
    if algorithmic:
        print(f"algorithmic_bytes: {algorithmic:.0f}  -> {algorithmic / (tot_us * 1e3):.1f} GB/s "
              f"over the kernel time")


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["trace", "pmc", "calib", "traffic", "table"])
    ap.add_argument("out_dir", type=Path, nargs="?")
    ap.add_argument("--kernel", default="")
    ap.add_argument("--kernels", default="")
    ap.add_argument("--bytes", type=int, default=0)
    ap.add_argument("--fetch", type=Path)
    ap.add_argument("--write", type=Path)
    ap.add_argument("--trace", type=Path)
    ap.add_argument("--calib-kernel", default="")
    ap.add_argument("--calib-bytes", type=int, default=0)
    ap.add_argument("--algorithmic-bytes", type=float, default=0.0)
    ap.add_argument("--near-us", type=float, default=0.0)
    a = ap.parse_args(argv)
    if a.mode == "table":
        table(a.fetch, a.write, a.trace, [k for k in a.kernels.split(",") if k], a.calib_kernel,
              a.calib_bytes, a.algorithmic_bytes)
    elif a.mode == "traffic":
        traffic(a.fetch, a.write, a.trace, a.kernel, a.calib_kernel, a.calib_bytes,
                a.algorithmic_bytes, a.near_us)
    elif a.mode == "trace":
        trace(a.out_dir)
    elif a.mode == "pmc":
        pmc(a.out_dir, a.kernel, a.trace, a.near_us)
    else:
        calib(a.out_dir, a.kernel, a.bytes)


if __name__ == "__main__":
    main(sys.argv[1:])
