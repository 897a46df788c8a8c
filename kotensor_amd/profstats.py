"""Summaries of rocprofv3 output (``--output-format csv``) for the performance record.

    python -m kotensor_amd.profstats stats DIR [PATTERN]
        per-kernel calls and average / min / max duration from a --kernel-trace run
    python -m kotensor_amd.profstats pmc DIR [PATTERN]
        per-kernel average of every counter per dispatch from a --pmc run
    python -m kotensor_amd.profstats traffic --kernel KDIR [KDIR2] --copy CDIR [CDIR2]
            --copy-bytes-read R --copy-bytes-written W --pattern P [--algorithmic B] [--out FILE]
        HBM bytes per launch of the kernels matching P: FETCH_SIZE and WRITE_SIZE (two runs
        each: one counter per run) scaled by what the same counters read for a device copy
        of known size; written as JSON (bytes_per_launch = read + written).

Only the CSV files rocprofv3 writes are read; nothing here touches the GPU.
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import os
import sys


def _files(root: str, suffix: str) -> list[str]:
    return sorted(glob.glob(os.path.join(root, "**", f"*{suffix}"), recursive=True))


def _col(header: list[str], *names: str) -> int:
    low = [h.lower() for h in header]
    for n in names:
        if n.lower() in low:
            return low.index(n.lower())
    raise KeyError(f"none of {names} in {header}")


def kernel_durations(root: str, pattern: str = "") -> dict[str, list[float]]:
    """'kernel name grid=XxY' -> durations in microseconds, from *_kernel_trace.csv (one
    entry per launch shape, so that products of different sizes stay apart)."""
    out: dict[str, list[float]] = collections.defaultdict(list)
    for path in _files(root, "kernel_trace.csv"):
        with open(path, newline="") as fh:
            rows = csv.reader(fh)
            header = next(rows)
            kn = _col(header, "Kernel_Name", "Name")
            st = _col(header, "Start_Timestamp", "Start")
            en = _col(header, "End_Timestamp", "End")
            try:
                gx, gy = _col(header, "Grid_Size_X"), _col(header, "Grid_Size_Y")
            except KeyError:
                gx = gy = None
            for r in rows:
                if pattern in r[kn]:
                    key = r[kn] if gx is None else f"{r[kn]} grid={r[gx]}x{r[gy]}"
                    out[key].append((int(r[en]) - int(r[st])) / 1000.0)
    return out


def counters(root: str, pattern: str = "") -> dict[str, dict[str, float]]:
    """Kernel name -> counter -> average value per dispatch, from *_counter_collection.csv."""
    per: dict[tuple[str, str], dict[str, float]] = collections.defaultdict(lambda: collections.defaultdict(float))
    for path in _files(root, "counter_collection.csv"):
        with open(path, newline="") as fh:
            rows = csv.reader(fh)
            header = next(rows)
            kn = _col(header, "Kernel_Name")
            di = _col(header, "Dispatch_Id")
            cn = _col(header, "Counter_Name")
            cv = _col(header, "Counter_Value")
            for r in rows:
                if pattern in r[kn]:
                    per[(r[kn], path + ":" + r[di])][r[cn]] += float(r[cv])
    by_kernel: dict[str, list[dict[str, float]]] = collections.defaultdict(list)
    for (name, _), vals in per.items():
        by_kernel[name].append(vals)
    result = {}
    for name, lst in by_kernel.items():
        keys = sorted({k for d in lst for k in d})
        result[name] = {k: sum(d.get(k, 0.0) for d in lst) / len(lst) for k in keys}
        result[name]["dispatches"] = float(len(lst))
    return result


def _short(name: str, width: int = 96) -> str:
    return name if len(name) <= width else name[: width - 3] + "..."


def _short_grid(name: str, width: int = 96) -> str:
    base, sep, grid = name.rpartition(" grid=")
    if not sep:
        return _short(name, width)
    tail = " grid=" + grid
    return _short(base, width - len(tail)) + tail


def cmd_stats(args) -> int:
    d = kernel_durations(args.dir, args.pattern)
    print(f"{'kernel (threads in grid)':96s} {'calls':>6s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s}")
    for name, v in sorted(d.items(), key=lambda kv: -sum(kv[1])):
        print(f"{_short_grid(name):96s} {len(v):6d} {sum(v) / len(v):9.3f} {min(v):9.3f} {max(v):9.3f}")
    return 0


def cmd_pmc(args) -> int:
    for name, vals in counters(args.dir, args.pattern).items():
        body = ", ".join(f"{k}={v:.6g}" for k, v in vals.items())
        print(f"{_short(name)} | {body}")
    return 0


def _one(root_list: list[str], pattern: str, counter: str) -> float:
    vals = []
    for root in root_list:
        for name, cs in counters(root, pattern).items():
            if counter in cs:
                vals.append(cs[counter])
    if not vals:
        raise SystemExit(f"no {counter} for kernels matching {pattern!r} under {root_list}")
    return sum(vals) / len(vals)


def cmd_traffic(args) -> int:
    # FETCH_SIZE / WRITE_SIZE read in KiB per dispatch; the copy gives the factor to bytes.
    k_fetch = _one(args.kernel, args.pattern, "FETCH_SIZE")
    k_write = _one(args.kernel, args.pattern, "WRITE_SIZE")
    c_fetch = _one(args.copy, args.copy_pattern, "FETCH_SIZE")
    c_write = _one(args.copy, args.copy_pattern, "WRITE_SIZE")
    f_read = args.copy_bytes_read / c_fetch
    f_write = args.copy_bytes_written / c_write
    read_b = k_fetch * f_read
    write_b = k_write * f_write
    out = {
        "kernel_pattern": args.pattern,
        "fetch_size_kib_per_dispatch": k_fetch,
        "write_size_kib_per_dispatch": k_write,
        "copy_fetch_size_kib": c_fetch,
        "copy_write_size_kib": c_write,
        "bytes_per_counter_unit_read": f_read,
        "bytes_per_counter_unit_write": f_write,
        "read_bytes_per_launch": round(read_b),
        "write_bytes_per_launch": round(write_b),
        "bytes_per_launch": round(read_b + write_b),
    }
    if args.algorithmic:
        out["algorithmic_bytes"] = args.algorithmic
        out["traffic_over_algorithmic"] = round((read_b + write_b) / args.algorithmic, 4)
    text = json.dumps(out, indent=2)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text + "\n")
    print(text)
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m kotensor_amd.profstats")
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("pattern", nargs="?", default="")
    p = sub.add_parser("pmc")
    p.add_argument("dir")
    p.add_argument("pattern", nargs="?", default="")
    t = sub.add_parser("traffic")
    t.add_argument("--kernel", nargs="+", required=True, help="PMC output dirs of the kernel (FETCH_SIZE, WRITE_SIZE)")
    t.add_argument("--copy", nargs="+", required=True, help="PMC output dirs of the calibration copy")
    t.add_argument("--copy-bytes-read", type=float, required=True)
    t.add_argument("--copy-bytes-written", type=float, required=True)
    t.add_argument("--pattern", required=True)
    # the calibration run's copy kernel only (its source buffer is filled by another kernel
    # first, whose counters must not enter the average)
    t.add_argument("--copy-pattern", default="copyBuffer")
    t.add_argument("--algorithmic", type=int, default=0)
    t.add_argument("--out", default="")
    args = ap.parse_args(argv)
    return {"stats": cmd_stats, "pmc": cmd_pmc, "traffic": cmd_traffic}[args.cmd](args)


if __name__ == "__main__":
    sys.exit(main())
