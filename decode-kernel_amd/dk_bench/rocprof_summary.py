"""Summarise rocprofv3 output (kernel trace or PMC counters) as short text.

    python decode-kernel_amd/dk_bench/rocprof_summary.py trace DIR [--kernel SUBSTR] [--runs N]
    python decode-kernel_amd/dk_bench/rocprof_summary.py pmc DIR [--kernel SUBSTR] [--json OUT]
                                                          [--sclk-mhz F]

Reads the CSV files rocprofv3 writes with `--output-format csv` (or, failing
that, the rocpd SQLite database) anywhere under DIR. `trace` prints per
kernel name and grid the dispatch count and the mean / p50 / min / max
duration; with `--runs N` it lists instead, in dispatch order, every run of
N or more consecutive dispatches of one kernel (so launches of one kernel at
different sizes, timed one after the other, stay apart). `pmc` prints the
mean counter value per dispatch and, when the d2d copy kernel of
profile_run.py (64 MiB read + 64 MiB written per launch) is present, the
factor that turns FETCH_SIZE / WRITE_SIZE into bytes and the scaled HBM bytes
per launch of every other kernel; with `--sclk-mhz F` counters kept in SCLK
cycles (SQ_BUSY_CYCLES and its DK_ max, GRBM_GUI_ACTIVE) are also given in
microseconds at F MHz (the clock profile_run.py --sclk prints in the same
run). Replaces the reference's
ncu wrapper (bench/ncu_collect.py:26-101).
"""

from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import sqlite3
import statistics
import sys
from collections import defaultdict

COPY_KERNEL = "stream_copy_kernel"
COPY_KIB = 64 * 1024  # 64 MiB each way per copy launch in profile_run.py


def _csvs(root: str, suffix: str) -> list[str]:
    return sorted(glob.glob(os.path.join(root, "**", f"*{suffix}"), recursive=True))


def _dbs(root: str) -> list[str]:
    return sorted(glob.glob(os.path.join(root, "**", "*.db"), recursive=True))


W = 92  # kernel name column


def _short(name: str, width: int = W) -> str:
    """The kernel name without its return type and parameter list (template
    arguments kept: they tell the launch shapes and the ablation maths
    apart), shortened in the middle if still too long."""
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0 and i > 0:
            name = name[:i]
            break
    if len(name) <= width:
        return name
    half = (width - 3) // 2
    return name[:half] + "..." + name[-(width - 3 - half):]


def load_trace(root: str) -> list[dict]:
    rows = []
    for path in _csvs(root, "kernel_trace.csv"):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                rows.append({
                    "name": r["Kernel_Name"],
                    "grid": int(r.get("Grid_Size_X") or r.get("Grid_Size", 0) or 0),
                    "start": int(r["Start_Timestamp"]),
                    "dur_ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"]),
                })
    if rows:
        return rows
    for path in _dbs(root):
        c = sqlite3.connect(path)
        for name, grid, start, end in c.execute("select name, grid_x, start, end from kernels"):
            rows.append({"name": name, "grid": int(grid or 0), "start": int(start),
                         "dur_ns": int(end) - int(start)})
    return rows


def load_pmc(root: str) -> list[dict]:
    rows = []
    for path in _csvs(root, "counter_collection.csv"):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                rows.append({
                    "name": r["Kernel_Name"], "dispatch": r.get("Dispatch_Id"),
                    "counter": r["Counter_Name"], "value": float(r["Counter_Value"]),
                })
    if rows:
        return rows
    for path in _dbs(root):
        c = sqlite3.connect(path)
        q = ("select kernel_name, dispatch_id, counter_name, value from counters_collection")
        try:
            for name, disp, cname, val in c.execute(q):
                rows.append({"name": name, "dispatch": disp, "counter": cname, "value": float(val)})
        except sqlite3.Error:
            continue
    return rows


def summarize_trace(rows: list[dict], match: str | None) -> str:
    groups = defaultdict(list)
    for r in rows:
        if match and match not in r["name"]:
            continue
        groups[(r["name"], r["grid"])].append(r["dur_ns"] / 1000.0)
    lines = [f"{'kernel':{W}s} {'grid':>9s} {'n':>5s} {'mean_us':>9s} {'p50_us':>9s} "
             f"{'min_us':>9s} {'max_us':>9s}"]
    for (name, grid), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        d.sort()
        lines.append(f"{_short(name):{W}s} {grid:9d} {len(d):5d} {statistics.fmean(d):9.2f} "
                     f"{d[len(d) // 2]:9.2f} {d[0]:9.2f} {d[-1]:9.2f}")
    return "\n".join(lines)


def summarize_runs(rows: list[dict], match: str | None, min_run: int) -> str:
    """Runs of >= min_run consecutive dispatches of one kernel and grid, in
    dispatch order, with the mean / p50 / min duration of each run."""
    rows = sorted(rows, key=lambda r: r["start"])
    runs = []
    for r in rows:
        key = (r["name"], r["grid"])
        if runs and runs[-1][0] == key:
            runs[-1][1].append(r["dur_ns"] / 1000.0)
        else:
            runs.append((key, [r["dur_ns"] / 1000.0]))
    lines = [f"{'run':>4s} {'kernel':{W}s} {'grid':>9s} {'n':>5s} {'mean_us':>9s} {'p50_us':>9s} "
             f"{'min_us':>9s}"]
    for i, ((name, grid), d) in enumerate(runs):
        if len(d) < min_run or (match and match not in name):
            continue
        d = sorted(d)
        lines.append(f"{i:4d} {_short(name):{W}s} {grid:9d} {len(d):5d} {statistics.fmean(d):9.2f} "
                     f"{d[len(d) // 2]:9.2f} {d[0]:9.2f}")
    return "\n".join(lines)


CYCLE_COUNTERS = ("DK_SQ_BUSY_CYCLES_max", "SQ_BUSY_CYCLES", "DK_GUI_ACTIVE_max", "GRBM_GUI_ACTIVE")


def summarize_pmc(rows: list[dict], match: str | None,
                  sclk_mhz: float | None = None) -> tuple[str, dict]:
    per = defaultdict(lambda: defaultdict(list))
    for r in rows:
        per[r["name"]][r["counter"]].append(r["value"])
    factors = {}
    for name, cs in per.items():
        if COPY_KERNEL in name:
            for cname in ("FETCH_SIZE", "WRITE_SIZE"):
                if cs.get(cname):
                    factors[cname] = COPY_KIB / statistics.fmean(cs[cname])
    lines = []
    if factors:
        lines.append("calibration (64 MiB d2d copy): " + ", ".join(
            f"{k} x{v:.4f}" for k, v in sorted(factors.items())))
    out = {}
    lines.append(f"{'kernel':{W}s} {'counter':22s} {'n':>5s} {'mean/dispatch':>14s} {'scaled bytes':>14s}")
    for name, cs in sorted(per.items()):
        if match and match not in name and COPY_KERNEL not in name:
            continue
        for cname, vals in sorted(cs.items()):
            m = statistics.fmean(vals)
            scaled = m * 1024 * factors[cname] if cname in factors else None
            out.setdefault(name, {})[cname] = {"mean_per_dispatch": m, "n": len(vals),
                                               "scaled_bytes": scaled}
            sb = f"{scaled:14.0f}" if scaled is not None else f"{'-':>14s}"
            extra = ""
            if sclk_mhz and cname in CYCLE_COUNTERS:
                extra = f"   = {m / sclk_mhz:.3f} us at {sclk_mhz:.0f} MHz"
                out[name][cname]["us_at_sclk"] = m / sclk_mhz
            lines.append(f"{_short(name):{W}s} {cname:22s} {len(vals):5d} {m:14.1f} {sb}{extra}")
    return "\n".join(lines), {"factors": factors, "kernels": out}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("mode", choices=["trace", "pmc"])
    ap.add_argument("root")
    ap.add_argument("--kernel", default=None, help="only kernels whose name contains this")
    ap.add_argument("--json", default=None, help="pmc: also write the numbers as JSON")
    ap.add_argument("--runs", type=int, default=0,
                    help="trace: list runs of at least this many consecutive dispatches")
    ap.add_argument("--sclk-mhz", type=float, default=None,
                    help="pmc: shader clock for converting cycle counters to microseconds")
    args = ap.parse_args()
    if args.mode == "trace":
        rows = load_trace(args.root)
        if not rows:
            print(f"no kernel trace under {args.root}", file=sys.stderr)
            return 1
        print(summarize_runs(rows, args.kernel, args.runs) if args.runs
              else summarize_trace(rows, args.kernel))
    else:
        rows = load_pmc(args.root)
        if not rows:
            print(f"no counter data under {args.root}", file=sys.stderr)
            return 1
        text, data = summarize_pmc(rows, args.kernel, args.sclk_mhz)
        print(text)
        if args.json:
            with open(args.json, "w") as f:
                json.dump(data, f, indent=2)
    return 0


if __name__ == "__main__":
    sys.exit(main())
