"""Per-kernel statistics from rocprofv3 output, as Markdown tables.  Companion of bench.py: the committed
profiles quote its output.

    python bench_trace_stats.py <dir>/**/<name>_kernel_trace.csv [--match REGEX] [--tail N]
        duration per dispatch: calls, average, median, minimum, maximum (ns);
        --tail N keeps only each kernel's last N dispatches (for bench.py --trace-headline, whose last
        launches are the timed graph replays);
        --runs: one row per run of consecutive matching dispatches of one kernel and grid size (a bench
        config that times several shapes of one kernel one after the other)
    python bench_trace_stats.py --counters <dir>/**/<name>_counter_collection.csv [--match REGEX]
        median value per dispatch of every counter (a kernel's dispatches summed per dispatch id)
"""
import argparse
import csv
import glob
import re
import statistics
import sys


def main():
    p = argparse.ArgumentParser()
    p.add_argument("trace", help="kernel_trace.csv path or glob")
    p.add_argument("--match", default="", help="only kernels whose name matches this regex")
    p.add_argument("--tail", type=int, default=0)
    p.add_argument("--runs", action="store_true")
    p.add_argument("--counters", action="store_true", help="the file is a counter_collection.csv")
    args = p.parse_args()
    if args.counters:
        return counters(args)
    paths = sorted(glob.glob(args.trace, recursive=True))
    if not paths:
        sys.exit(f"no trace file matches {args.trace}")
    rows = []
    for path in paths:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"],
                             r.get("Grid_Size_X", "")))
    rows.sort()
    if args.runs:
        return runs(args, rows)
    per = {}
    for s, e, name, _ in rows:
        if args.match and not re.search(args.match, name):
            continue
        per.setdefault(name, []).append(e - s)
    print("| kernel | calls | avg ns | median ns | min ns | max ns |")
    print("|---|---|---|---|---|---|")
    for name, d in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        if args.tail:
            d = d[-args.tail:]
        print(f"| `{name[:110]}` | {len(d)} | {statistics.mean(d):.0f} | {statistics.median(d):.0f} | {min(d)} | "
              f"{max(d)} |")


def runs(args, rows):
    out = []  # [(name, grid, durations)]
    for s, e, name, grid in rows:
        if args.match and not re.search(args.match, name):
            continue
        if out and out[-1][0] == name and out[-1][1] == grid:
            out[-1][2].append(e - s)
        else:
            out.append((name, grid, [e - s]))
    print("| kernel | grid | calls | avg ns | median ns | min ns | max ns |")
    print("|---|---|---|---|---|---|---|")
    for name, grid, d in out:
        print(f"| `{name[:110]}` | {grid} | {len(d)} | {statistics.mean(d):.0f} | {statistics.median(d):.0f} | "
              f"{min(d)} | {max(d)} |")


def counters(args):
    per = {}  # kernel -> counter -> dispatch id -> value
    for path in sorted(glob.glob(args.trace, recursive=True)):
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                name = r["Kernel_Name"]
                if args.match and not re.search(args.match, name):
                    continue
                d = per.setdefault(name, {}).setdefault(r["Counter_Name"], {})
                d[r["Dispatch_Id"]] = d.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    names = sorted({c for k in per.values() for c in k})
    print("| kernel | dispatches | " + " | ".join(names) + " |")
    print("|---|---|" + "---|" * len(names))
    for kern, cs in sorted(per.items(), key=lambda kv: -max(len(v) for v in kv[1].values())):
        n = max(len(v) for v in cs.values())
        vals = [f"{statistics.median(cs[c].values()):,.1f}" if c in cs else "" for c in names]
        print(f"| `{kern[:90]}` | {n} | " + " | ".join(vals) + " |")


if __name__ == "__main__":
    main()
