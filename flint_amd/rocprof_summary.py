"""Condense a `rocprofv3 --kernel-trace --stats -f csv` run into the short text kept under profiles/.

    python -m flint_amd.rocprof_summary <rocprof output dir> [--kernel k_decode] [--last N]

Prints the per-kernel stats table (calls, total, average, min, max) and, for the named kernel,
the average duration of its last N dispatches (the timed window of a bench run, whose earlier
dispatches are prefill / warmup at other context lengths).
"""
import argparse
import csv
import glob
import os
import sys


def _find(d, suffix):
    hits = sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {d}")
    return hits[-1]


def _short(name, width=60):
    name = name.replace("(anonymous namespace)::", "")
    return name if len(name) <= width else name[: width - 3] + "..."


def summarise(d, kernel="k_decode", last=0, top=8):
    out = []
    stats = _find(d, "kernel_stats.csv")
    with open(stats) as f:
        rows = list(csv.DictReader(f))
    out.append(f"kernel stats ({os.path.basename(stats)}), top {top} by total time:")
    out.append(f"{'kernel':60s} {'calls':>7s} {'total_ms':>10s} {'avg_us':>9s} {'min_us':>9s} "
               f"{'max_us':>9s} {'pct':>6s}")
    for r in rows[:top]:
        out.append(f"{_short(r['Name']):60s} {int(r['Calls']):7d} {float(r['TotalDurationNs']) / 1e6:10.3f} "
                   f"{float(r['AverageNs']) / 1e3:9.2f} {float(r['MinNs']) / 1e3:9.2f} "
                   f"{float(r['MaxNs']) / 1e3:9.2f} {float(r['Percentage']):6.2f}")
    trace = _find(d, "kernel_trace.csv")
    with open(trace) as f:
        disp = [r for r in csv.DictReader(f) if kernel in r["Kernel_Name"]]
    disp.sort(key=lambda r: int(r["Start_Timestamp"]))
    durs = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in disp]
    if durs:
        win = durs[-last:] if last else durs
        out.append("")
        out.append(f"{kernel}: {len(durs)} dispatches; last {len(win)} (timed window): "
                   f"avg {sum(win) / len(win):.2f} us, min {min(win):.2f} us, max {max(win):.2f} us")
        if len(disp) > 1:
            s = [int(r["Start_Timestamp"]) for r in disp[-len(win):]]
            e = [int(r["End_Timestamp"]) for r in disp[-len(win):]]
            gaps = [(s[i + 1] - e[i]) / 1e3 for i in range(len(s) - 1)]
            if gaps:
                out.append(f"{kernel}: idle gap between consecutive timed dispatches: avg "
                           f"{sum(gaps) / len(gaps):.2f} us")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("dir")
    ap.add_argument("--kernel", default="k_decode")
    ap.add_argument("--last", type=int, default=0)
    a = ap.parse_args(argv)
    print(summarise(a.dir, a.kernel, a.last))


if __name__ == "__main__":
    sys.exit(main())
