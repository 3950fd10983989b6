"""Readers for rocprofv3 output, used to build the summaries under profiles/.

    python -m foundry_amd.profiling stats <dir>        # kernel-trace --stats CSV
    python -m foundry_amd.profiling trace <dir>        # per-dispatch medians from the kernel trace
    python -m foundry_amd.profiling counters <dir> <kernel-substring>   # --pmc values per dispatch
    python -m foundry_amd.profiling traffic <fetch_dir> <write_dir> <kernel-substring> [grid-size]

``traffic`` takes two ``rocprofv3 --pmc`` runs of the same command, one with
FETCH_SIZE and one with WRITE_SIZE (KiB per dispatch), each of which also ran
``bench.py --calibrate-copy`` (a device-to-device copy of a known byte count).
Each counter is scaled by known bytes / what the counter read for the copy
kernel, then averaged over the dispatches of the named kernel (of the given
total grid size, in work-items, when one is given).
"""
from __future__ import annotations

import csv
import glob
import os
import statistics
import sys

COPY_KERNEL = "copyBuffer"
CALIBRATION_BYTES = 256 << 20  # bench.py --calibrate-copy copies this many bytes


def _rows(pattern: str):
    for path in glob.glob(pattern, recursive=True):
        with open(path, newline="") as f:
            yield from csv.DictReader(f)


def kernel_stats(directory: str):
    """[(name, calls, avg_ns, total_ns)] from a *_kernel_stats.csv."""
    out = []
    for r in _rows(os.path.join(directory, "**", "*kernel_stats.csv")):
        out.append((r["Name"], int(r["Calls"]), float(r["AverageNs"]), float(r["TotalDurationNs"])))
    return sorted(out, key=lambda t: -t[3])


def trace_medians(directory: str):
    """[(name, grid, block, dispatches, median_us, mean_us, total_ms)] from
    the per-dispatch rows of a *_kernel_trace.csv, grouped by kernel and
    grid."""
    groups = {}
    for r in _rows(os.path.join(directory, "**", "*kernel_trace.csv")):
        key = (r["Kernel_Name"], f'{r["Grid_Size_X"]} x {r["Grid_Size_Y"]} x {r["Grid_Size_Z"]}',
               r["Workgroup_Size_X"])
        groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    out = [(k[0], k[1], k[2], len(v), statistics.median(v), statistics.mean(v), sum(v) / 1e3)
           for k, v in groups.items()]
    return sorted(out, key=lambda t: -t[6])


def counters_by_kernel(directory: str, kernel_substring: str):
    """{(kernel, grid size): {counter: (mean value per dispatch, dispatches)}}
    over the dispatches of the kernels whose name contains the substring."""
    acc = {}
    for r in _rows(os.path.join(directory, "**", "*counter_collection.csv")):
        if kernel_substring in r["Kernel_Name"]:
            key = (r["Kernel_Name"].split("(")[0], r["Grid_Size"])
            acc.setdefault(key, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    return {k: {c: (statistics.mean(v), len(v)) for c, v in d.items()} for k, d in acc.items()}


def counter_per_dispatch(directory: str, counter: str, kernel_substring: str, grid: str | None = None):
    vals = [float(r["Counter_Value"]) for r in _rows(os.path.join(directory, "**", "*counter_collection.csv"))
            if r["Counter_Name"] == counter and kernel_substring in r["Kernel_Name"]
            and (grid is None or r["Grid_Size"] == grid)]
    return vals


def scaled_bytes(directory: str, counter: str, kernel_substring: str, grid: str | None = None):
    """Mean bytes per dispatch of the kernel, scaled by the copy calibration."""
    kernel = counter_per_dispatch(directory, counter, kernel_substring, grid)
    copy = counter_per_dispatch(directory, counter, COPY_KERNEL)
    if not kernel or not copy:
        raise RuntimeError(f"{counter}: no dispatches of {kernel_substring!r} or of the copy kernel in {directory}")
    # the copy reads and writes CALIBRATION_BYTES each
    scale = CALIBRATION_BYTES / (max(copy) * 1024.0)
    return statistics.mean(kernel) * 1024.0 * scale, scale, len(kernel)


def main(argv):
    if len(argv) >= 2 and argv[0] == "stats":
        for name, calls, avg, total in kernel_stats(argv[1]):
            print(f"| {name[:90]} | {calls} | {avg / 1e3:.2f} | {total / 1e6:.3f} |")
        return 0
    if len(argv) >= 2 and argv[0] == "trace":
        print("| Kernel | grid | block | dispatches | median us | mean us | total ms |")
        print("|---|---|---|---|---|---|---|")
        for name, grid, block, n, med, mean, total in trace_medians(argv[1]):
            short = name.split("(")[0][:80]
            print(f"| `{short}` | {grid} | {block} | {n} | {med:.2f} | {mean:.2f} | {total:.3f} |")
        return 0
    if len(argv) >= 3 and argv[0] == "counters":
        for (kernel, grid), d in sorted(counters_by_kernel(argv[1], argv[2]).items()):
            print(f"{kernel} (grid {grid}):")
            for name, (mean, n) in sorted(d.items()):
                print(f"  {name}={mean:.6g} (mean of {n} dispatches)")
        return 0
    if len(argv) >= 4 and argv[0] == "traffic":
        grid = argv[4] if len(argv) >= 5 else None
        fetch, fscale, n1 = scaled_bytes(argv[1], "FETCH_SIZE", argv[3], grid)
        write, wscale, n2 = scaled_bytes(argv[2], "WRITE_SIZE", argv[3], grid)
        print(f"fetch_bytes_per_dispatch={fetch:.0f} (scale {fscale:.4f}, {n1} dispatches)")
        print(f"write_bytes_per_dispatch={write:.0f} (scale {wscale:.4f}, {n2} dispatches)")
        print(f"traffic_bytes_per_dispatch={fetch + write:.0f}")
        return 0
    print(__doc__)
    return 2


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
