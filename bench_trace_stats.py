"""Per-kernel duration statistics (calls, average, median, minimum, maximum in ns) from a rocprofv3
kernel trace, as a Markdown table.  Companion of bench.py: the committed profiles quote its output.

    python bench_trace_stats.py <dir>/**/<name>_kernel_trace.csv [--match REGEX] [--tail N]

--tail N keeps only each kernel's last N dispatches (for bench.py --trace-headline, whose last launches
are the timed graph replays).
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
    args = p.parse_args()
    paths = sorted(glob.glob(args.trace, recursive=True))
    if not paths:
        sys.exit(f"no trace file matches {args.trace}")
    rows = []
    for path in paths:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    per = {}
    for s, e, name in rows:
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


if __name__ == "__main__":
    main()
