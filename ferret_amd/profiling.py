"""Summaries of rocprofv3 CSV output for the profiles/ directory.

    python -m ferret_amd.profiling trace  <kernel_trace.csv>            # per (kernel, grid) durations
    python -m ferret_amd.profiling traffic <kernel substring> <fetch_dir> <write_dir> \\
        <copy_fetch_dir> <copy_write_dir> <copy_bytes>                  # HBM bytes per launch
    python -m ferret_amd.profiling counters <kernel substring> <pmc_dir> [<pmc_dir> ...]
                                                                        # median per dispatch of each counter

FETCH_SIZE / WRITE_SIZE are read in KiB per dispatch and scaled by what the
same counter reads for a plain device copy of known size (the calibration
factor), as `bench.py --copy-bytes` produces it.
"""
from __future__ import annotations

import csv
import glob
import json
import os
import statistics
import sys
from collections import defaultdict


def _rows(path: str):
    if os.path.isdir(path):
        path = glob.glob(os.path.join(path, "*counter_collection.csv"))[0]
    with open(path) as fh:
        return list(csv.DictReader(fh))


def kernel_table(trace_csv: str, match: str = "ferret") -> list[dict]:
    groups = defaultdict(list)
    for r in _rows(trace_csv):
        name = r["Kernel_Name"]
        if match and match not in name:
            continue
        grid = r.get("Grid_Size") or r.get("Grid_Size_X") or "?"
        groups[(name, grid)].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    out = []
    for (name, grid), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        out.append({"kernel": name, "grid": grid, "calls": len(d), "avg_us": statistics.mean(d),
                    "min_us": min(d), "max_us": max(d)})
    return out


def counter_per_dispatch(path: str, kernel_substr: str) -> float:
    vals = [float(r["Counter_Value"]) for r in _rows(path) if kernel_substr in r["Kernel_Name"]]
    if not vals:
        raise ValueError(f"no dispatch of {kernel_substr!r} in {path}")
    return statistics.median(vals)


def counters(kernel_substr: str, path: str) -> dict[str, float]:
    """Median per dispatch of every counter a rocprofv3 --pmc run recorded for the kernel."""
    vals = defaultdict(list)
    for r in _rows(path):
        if kernel_substr in r["Kernel_Name"]:
            vals[r["Counter_Name"]].append(float(r["Counter_Value"]))
    if not vals:
        raise ValueError(f"no dispatch of {kernel_substr!r} in {path}")
    return {k: statistics.median(v) for k, v in sorted(vals.items())}


def copy_factors(copy_fetch_dir: str, copy_write_dir: str, copy_bytes: int) -> tuple[float, float]:
    """Bytes per counted KiB of FETCH_SIZE and WRITE_SIZE, from a device copy of copy_bytes."""
    kib = copy_bytes / 1024.0
    return (kib / counter_per_dispatch(copy_fetch_dir, "copyBuffer"),
            kib / counter_per_dispatch(copy_write_dir, "copyBuffer"))


def traffic(kernel_substr: str, fetch_dir: str, write_dir: str, copy_fetch_dir: str, copy_write_dir: str,
            copy_bytes: int, factors: tuple[float, float] | None = None) -> dict:
    """HBM bytes per launch of the kernel; `factors` (from copy_factors) skips
    reading the copy runs again."""
    f_factor, w_factor = factors or copy_factors(copy_fetch_dir, copy_write_dir, copy_bytes)
    fetch = counter_per_dispatch(fetch_dir, kernel_substr) * f_factor * 1024
    write = counter_per_dispatch(write_dir, kernel_substr) * w_factor * 1024
    return {"fetch_bytes": round(fetch), "write_bytes": round(write), "bytes_per_launch": round(fetch + write),
            "fetch_factor": round(f_factor, 4), "write_factor": round(w_factor, 4)}


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if argv and argv[0] == "trace":
        print("| kernel | grid | calls | avg us | min us | max us |\n|---|---|---|---|---|---|")
        for r in kernel_table(argv[1]):
            print(f"| `{r['kernel'][:90]}` | {r['grid']} | {r['calls']} | {r['avg_us']:.2f} | "
                  f"{r['min_us']:.2f} | {r['max_us']:.2f} |")
        return 0
    if argv and argv[0] == "counters":
        print("| counter | median per dispatch |\n|---|---|")
        for d in argv[2:]:
            for name, v in counters(argv[1], d).items():
                print(f"| {name} | {v:,.0f} |")
        return 0
    if argv and argv[0] == "traffic":
        print(json.dumps(traffic(argv[1], argv[2], argv[3], argv[4], argv[5], int(argv[6]))))
        return 0
    print(__doc__)
    return 2


if __name__ == "__main__":
    raise SystemExit(main())
