"""Markdown summaries of rocprofv3 CSV output for the library's kernels.

    python -m gaussian_splatting.rasterizer.rocprof_summary trace <dir>
        kernel table from `rocprofv3 --kernel-trace --stats ... --output-format csv -d <dir> -o run`
    python -m gaussian_splatting.rasterizer.rocprof_summary traffic <fetch_dir> <write_dir> --copy-bytes B
        HBM bytes per dispatch from a `--pmc FETCH_SIZE` and a `--pmc WRITE_SIZE` run. Each counter is
        scaled by what it reads for the run's plain device-to-device copy of B bytes (bench.py
        --calibrate-copy-mib), so the figures are in the bytes that copy is known to move.
    python -m gaussian_splatting.rasterizer.rocprof_summary mfma <label>=<dir> ... [--kernels K ...]
        matrix-core use per dispatch from `--pmc MfmaUtil MfmaFlopsBF16` runs: the share of cycles the
        MFMA pipes are busy (rocprofv3's MfmaUtil, percent of SIMD cycles) and the bf16 MFMA rate
        against MI355X's dense 2.5 PFLOP/s, one row per (label, kernel).

Kernel names are shortened to the function name without template arguments.
"""
from __future__ import annotations

import argparse
import collections
import csv
import re
import sys
from pathlib import Path


def short_name(name: str) -> str:
    name = name.replace("(anonymous namespace)::", "").replace("void ", "")
    if name.startswith("at::"):
        return name[:60]
    return re.sub(r"<.*", "", name.split("(")[0])


def trace(directory: Path, top: int) -> str:
    rows = list(csv.DictReader(open(next(directory.glob("*kernel_stats.csv")))))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    out = ["| kernel | calls | avg us | total ms | % |", "|---|---:|---:|---:|---:|"]
    for r in rows[:top]:
        out.append(f"| {short_name(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                   f"{float(r['TotalDurationNs']) / 1e6:.3f} | {100 * float(r['TotalDurationNs']) / total:.2f} |")
    out.append(f"\nAll kernels: {total / 1e6:.3f} ms.")
    spans = concurrent_spans(directory, "backward_geometry_kernel", "backward_features_kernel")
    if spans:
        out.append(f"\nbackward_geometry_kernel and backward_features_kernel run side by side: over {len(spans)} "
                   f"calls, first start to last end averages {sum(spans) / len(spans) / 1e3:.1f} us.")
    return "\n".join(out)


def concurrent_spans(directory: Path, first: str, second: str) -> list[int]:
    """Per call, the time from the earlier start to the later end of two kernels launched together
    (each dispatch of `first` paired with the `second` dispatch that starts nearest to it), in ns."""
    files = list(directory.glob("*kernel_trace.csv"))
    if not files:
        return []
    rows = list(csv.DictReader(open(files[0])))
    a = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in rows if short_name(r["Kernel_Name"]) == first]
    b = [(int(r["Start_Timestamp"]), int(r["End_Timestamp"])) for r in rows if short_name(r["Kernel_Name"]) == second]
    spans = []
    for s0, e0 in a:
        if not b:
            break
        s1, e1 = min(b, key=lambda se: abs(se[0] - s0))
        spans.append(max(e0, e1) - min(s0, s1))
    return spans


def _counter_values(directory: Path, counter: str) -> dict[str, list[float]]:
    """Counter values per kernel in dispatch order."""
    rows = [r for r in csv.DictReader(open(next(directory.glob("*counter_collection.csv"))))
            if r["Counter_Name"] == counter]
    values = collections.defaultdict(list)
    for r in sorted(rows, key=lambda r: int(r["Dispatch_Id"])):
        values[short_name(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    return values


def traffic(fetch_dir: Path, write_dir: Path, copy_bytes: int, kernels: list[str]) -> str:
    fetch_all = _counter_values(fetch_dir, "FETCH_SIZE")
    write_all = _counter_values(write_dir, "WRITE_SIZE")
    copy = [k for k in fetch_all if "copyBuffer" in k]
    if not copy:
        raise SystemExit("no copy kernel in the FETCH_SIZE run: run bench.py with --calibrate-copy-mib")
    # The calibration copy is the run's last copy dispatch (bench.py makes it after everything else).
    copy_fetch, copy_write = fetch_all[copy[0]][-1], write_all[copy[0]][-1]
    f_scale = copy_bytes / copy_fetch
    w_scale = copy_bytes / copy_write
    fetch = {k: sum(v) / len(v) for k, v in fetch_all.items()}
    write = {k: sum(v) / len(v) for k, v in write_all.items()}
    out = [f"Calibration: the last `{copy[0]}` dispatch copies {copy_bytes} bytes and reads FETCH_SIZE "
           f"{copy_fetch:.0f}, WRITE_SIZE {copy_write:.0f}, so one counter unit is {f_scale:.1f} bytes read / "
           f"{w_scale:.1f} bytes written. Figures are means per dispatch.", "",
           "| kernel | FETCH_SIZE | WRITE_SIZE | fetch bytes | write bytes | traffic_bytes |",
           "|---|---:|---:|---:|---:|---:|"]
    names = kernels or sorted(set(fetch) & set(write), key=lambda k: -(fetch[k] + write[k]))
    for k in names:
        if k not in fetch or k not in write or "copyBuffer" in k:
            continue
        fb, wb = fetch[k] * f_scale, write[k] * w_scale
        out.append(f"| {k} | {fetch[k]:.0f} | {write[k]:.0f} | {fb:.0f} | {wb:.0f} | {int(round(fb + wb))} |")
    return "\n".join(out)


MFMA_BF16_PEAK_TFLOPS = 2500.0


def mfma(runs: list[tuple[str, Path]], kernels: list[str]) -> str:
    out = ["| run | kernel | dispatches | MFMA busy % | bf16 TFLOP/s | of 2.5 PFLOP/s |", "|---|---|---:|---:|---:|---:|"]
    for label, directory in runs:
        rows = list(csv.DictReader(open(next(directory.glob("*counter_collection.csv")))))
        per = collections.defaultdict(lambda: collections.defaultdict(list))
        for r in rows:
            k = short_name(r["Kernel_Name"])
            if kernels and k not in kernels:
                continue
            per[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
            per[k]["ns"].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        for k, c in per.items():
            util, flops = c.get("MfmaUtil", []), c.get("MfmaFlopsBF16", [])
            if not util or not flops:
                continue
            ns = sum(c["ns"]) / len(c["ns"])
            rate = (sum(flops) / len(flops)) / ns / 1e3  # TFLOP/s
            out.append(f"| {label} | {k} | {len(util)} | {sum(util) / len(util):.1f} | {rate:.1f} | "
                       f"{rate / MFMA_BF16_PEAK_TFLOPS:.3f} |")
    return "\n".join(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir", type=Path)
    t.add_argument("--top", type=int, default=20)
    f = sub.add_parser("traffic")
    f.add_argument("fetch_dir", type=Path)
    f.add_argument("write_dir", type=Path)
    f.add_argument("--copy-bytes", type=int, required=True)
    f.add_argument("--kernels", nargs="*", default=[])
    m = sub.add_parser("mfma")
    m.add_argument("runs", nargs="+", help="label=directory")
    m.add_argument("--kernels", nargs="*", default=[])
    args = ap.parse_args(argv)
    if args.cmd == "trace":
        print(trace(args.dir, args.top))
    elif args.cmd == "mfma":
        runs = [(r.split("=", 1)[0], Path(r.split("=", 1)[1])) for r in args.runs]
        print(mfma(runs, args.kernels))
    else:
        print(traffic(args.fetch_dir, args.write_dir, args.copy_bytes, args.kernels))
    return 0


if __name__ == "__main__":
    sys.exit(main())
