"""Condense rocprofv3 CSV output into the short text kept under profiles/.

    python -m flint_amd.rocprof_summary <dir> [--kernel k_decode] [--last N] [--skip-last S] [--by-grid]
        from `rocprofv3 --kernel-trace --stats -f csv`: the per-kernel stats table and, for the
        named kernel, the average duration of its last N dispatches (the timed window of a
        bench run, whose earlier dispatches are prefill / warmup at other context lengths);
    python -m flint_amd.rocprof_summary --pmc <dir> [<dir> ...] --kernel k_decode --last N
        from `rocprofv3 --pmc ...` runs: every counter's mean per dispatch over the kernel's last N
        dispatches, and the same counters for the last device copy (copyBuffer) if there is one;
    python -m flint_amd.rocprof_summary --gemv <trace dir> <SQ pmc dir> <fetch dir> <write dir> --copy-bytes B
        the config-1 GEMV sweep (bench.py --gemv-only --no-steady --copy-probe-mb M): per kernel variant and
        shape the kernel time, algorithmic and HBM bytes, VALU issue and wait shares;
    python -m flint_amd.rocprof_summary --traffic <fetch dir> <write dir> --copy-bytes B ...
        from two `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE` runs of a bench command that
        ends with a device-to-device copy of B bytes: HBM bytes per dispatch of the kernel, each
        counter scaled by what it reads for the copy (which reads B and writes B bytes).
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


def summarise(d, kernel="k_decode", last=0, top=8, skip_last=0, by_grid=False):
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
    if skip_last:  # leave out the last skip_last dispatches (a later window of the same kernel)
        disp = disp[:-skip_last]
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
        if by_grid:  # one line per launch shape (grid size) in the window
            groups = {}
            for r, dur in zip(disp[-len(win):], win):
                groups.setdefault(int(r["Grid_Size_X"]), []).append(dur)
            for gx in sorted(groups):
                v = groups[gx]
                out.append(f"{kernel}: grid {gx}: {len(v)} dispatches, avg {sum(v) / len(v):.2f} us, "
                           f"min {min(v):.2f} us, max {max(v):.2f} us")
    return "\n".join(out)


def _counter_rows(d):
    path = _find(d, "counter_collection.csv")
    with open(path) as f:
        return path, list(csv.DictReader(f))


def _per_dispatch(rows, pattern):
    vals = {}
    for r in rows:
        if pattern in r["Kernel_Name"]:
            k = int(r.get("Dispatch_Id") or r.get("Correlation_Id") or 0)
            vals[k] = vals.get(k, 0.0) + float(r["Counter_Value"])
    return [vals[k] for k in sorted(vals)]


def pmc(dirs, kernel, last, copy_kernel="copyBuffer"):
    out = []
    for d in dirs:
        path, rows = _counter_rows(d)
        per, names = {}, {}
        for r in rows:
            k = int(r.get("Dispatch_Id") or r.get("Correlation_Id") or 0)
            names[k] = r["Kernel_Name"]
            c = per.setdefault(k, {})
            c[r["Counter_Name"]] = c.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        ks = [k for k in sorted(per) if kernel in names[k]]
        ks = ks[-last:] if last else ks
        if not ks:
            raise RuntimeError(f"no {kernel} dispatches in {path}")
        out.append(f"{os.path.basename(path)}: {kernel}, mean of last {len(ks)} dispatches")
        for cn in sorted(per[ks[0]]):
            out.append(f"  {cn:28s} {sum(per[k][cn] for k in ks) / len(ks):18.1f}")
        cp = [k for k in sorted(per) if copy_kernel in names[k]]
        if cp:
            out.append(f"  (device copy, {copy_kernel}):")
            for cn in sorted(per[cp[-1]]):
                out.append(f"  {cn:28s} {per[cp[-1]][cn]:18.1f}")
    return "\n".join(out)


def traffic(fetch_dir, write_dir, kernel, last, copy_bytes, config, copy_kernel="copyBuffer"):
    out = [f"config: {config}"]
    tot = 0.0
    for name, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        path, rows = _counter_rows(d)
        k = _per_dispatch(rows, kernel)
        c = _per_dispatch(rows, copy_kernel)
        if not k or not c:
            raise RuntimeError(f"{name}: no {kernel} or {copy_kernel} dispatches in {path}")
        win = k[-last:] if last else k
        kib = sum(win) / len(win)
        factor = c[-1] * 1024.0 / copy_bytes  # counter bytes per byte the copy moved
        bytes_ = kib * 1024.0 / factor
        tot += bytes_
        out.append(f"{name}_kib_per_dispatch: {kib:.1f}  (mean of last {len(win)} of {len(k)})")
        out.append(f"{name}_copy_kib: {c[-1]:.1f}  (copy of {copy_bytes} bytes; scale {factor:.4f})")
        out.append(f"{name}_bytes_per_launch: {bytes_:.0f}")
    out.append(f"traffic_bytes_per_launch: {tot:.0f}")
    return "\n".join(out)


def _gemv_label(name, grid, seen):
    """(variant, shape) of a config-1 GEMV dispatch from bench.gemv_sweep (run with --no-steady):
    the streamed row-layout kernel (template <4, 5>: K 2560; <6, 4>: K 8192) and the tiled
    matrix-core kernel (k_gemv_tiled_pf <4, 8>: K 2560; <8, 8>: K 8192; the older k_gemv_tiled:
    O and down share a grid and alternate, O first), told apart by kernel name and grid."""
    if "k_gemv_stream<4, 5>" in name:
        return "stream", {57344: "qkv", 40960: "o", 131072: "gate_up", 262144: "gate_up"}.get(grid)
    if "k_gemv_stream<6, 4>" in name:
        return "stream", "down"
    if "k_gemv_tiled_pf<8, 8>" in name:
        return "tiled", "down"
    if "k_gemv_tiled_pf<4, 8>" in name:
        return "tiled", {57344: "qkv", 40960: "o", 262144: "gate_up"}.get(grid)
    if "k_gemv_tiled" in name:
        if grid == 40960:
            seen["t40960"] = seen.get("t40960", 0) + 1
            return "tiled", "o" if seen["t40960"] % 2 == 1 else "down"
        return "tiled", {57344: "qkv", 262144: "gate_up"}.get(grid)
    return None, None


GEMV_SHAPES = {"qkv": (3584, 2560), "o": (2560, 2560), "gate_up": (16384, 2560), "down": (2560, 8192)}
SIMDS, CLOCK_HZ = 256 * 4, 2.4e9  # MI355X: 256 CUs of 4 SIMDs, 2.4 GHz peak engine clock


def gemv(trace_dir, pmc_dir, fetch_dir, write_dir, copy_bytes, skip_frac=0.25):
    """Config-1 GEMV table: per kernel variant and shape, the kernel time (trace), the algorithmic
    and HBM (FETCH + WRITE, copy-calibrated) bytes, and the PMC counters' story (VALU issue share,
    waiting share). The first skip_frac of each series (the sweep's warm-up pass) is left out."""
    out = []
    series = {}
    with open(_find(trace_dir, "kernel_trace.csv")) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    seen = {}
    for r in rows:
        v, shp = _gemv_label(r["Kernel_Name"], int(r["Grid_Size_X"]), seen)
        if v and shp:
            series.setdefault((v, shp), []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)

    def counters(d):
        _, crow = _counter_rows(d)
        per, meta = {}, {}
        for r in crow:
            k = int(r["Dispatch_Id"])
            meta[k] = (r["Kernel_Name"], int(r["Grid_Size"]))
            per.setdefault(k, {})[r["Counter_Name"]] = per.setdefault(k, {}).get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        res, sn = {}, {}
        for k in sorted(per):
            v, shp = _gemv_label(meta[k][0], meta[k][1], sn)
            if v and shp:
                res.setdefault((v, shp), []).append(per[k])
        copy = [per[k] for k in sorted(per) if "copyBuffer" in meta[k][0]]
        return res, (copy[-1] if copy else None)

    def mean(lst, key):
        lst = lst[int(len(lst) * skip_frac):]
        return sum(x[key] for x in lst) / len(lst)
    sq, _ = counters(pmc_dir)
    fe, fcopy = counters(fetch_dir)
    wr, wcopy = counters(write_dir)
    fscale = fcopy["FETCH_SIZE"] * 1024.0 / copy_bytes
    wscale = wcopy["WRITE_SIZE"] * 1024.0 / copy_bytes
    out.append(f"FETCH_SIZE reads {fscale:.4f}x and WRITE_SIZE {wscale:.4f}x the bytes of a {copy_bytes}-byte "
               f"device copy (the scale applied below)")
    out.append(f"{'variant':8s} {'shape':8s} {'kernel_us':>9s} {'alg_MB':>8s} {'hbm_MB':>8s} {'GB/s':>7s} {'frac':>6s} "
               f"{'VALU%':>6s} {'wait%':>6s} {'VALU/wt':>7s} {'VALU_us':>7s}")
    for (v, shp) in sorted(series, key=lambda t: (t[0], list(GEMV_SHAPES).index(t[1]))):
        n, k = GEMV_SHAPES[shp]
        t = series[(v, shp)]
        t = t[int(len(t) * skip_frac):]
        us = sum(t) / len(t)
        alg = n * k // 2 + n * (k // 128) * 4 + 2 * k + 2 * n
        hbm = (mean(fe[(v, shp)], "FETCH_SIZE") * 1024.0 / fscale + mean(wr[(v, shp)], "WRITE_SIZE") * 1024.0 / wscale)
        c = sq[(v, shp)]
        waves = mean(c, "SQ_WAVES")
        wave_cyc = mean(c, "SQ_WAVE_CYCLES") / waves
        valu = mean(c, "SQ_ACTIVE_INST_VALU") / waves / wave_cyc   # VALU busy share of a wave's life
        wait = mean(c, "SQ_WAIT_INST_ANY") / waves / wave_cyc
        per_w = mean(c, "SQ_INSTS_VALU") * 64.0 / (n * k)          # VALU lane-ops per weight
        # the VALU floor: every wave64 VALU instruction takes at least 4 cycles of its SIMD (16
        # lanes), spread over MI355X's 1024 SIMDs at the 2.4 GHz peak clock
        valu_us = mean(c, "SQ_INSTS_VALU") * 4.0 / (SIMDS * CLOCK_HZ) * 1e6
        gbs = alg / (us * 1e-6) / 1e9
        out.append(f"{v:8s} {shp:8s} {us:9.2f} {alg / 1e6:8.2f} {hbm / 1e6:8.2f} {gbs:7.0f} {gbs / 8000.0:6.3f} "
                   f"{100 * valu:6.1f} {100 * wait:6.1f} {per_w:7.2f} {valu_us:7.2f}")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("dir", nargs="*")
    ap.add_argument("--kernel", default="k_decode")
    ap.add_argument("--last", type=int, default=0)
    ap.add_argument("--skip-last", type=int, default=0)
    ap.add_argument("--by-grid", action="store_true", help="also one line per grid size")
    ap.add_argument("--traffic", action="store_true")
    ap.add_argument("--pmc", action="store_true")
    ap.add_argument("--copy-bytes", type=int, default=0)
    ap.add_argument("--config", default="")
    ap.add_argument("--gemv", action="store_true",
                    help="config-1 GEMV table from <trace dir> <SQ pmc dir> <FETCH dir> <WRITE dir>")
    a = ap.parse_args(argv)
    if a.gemv:
        print(gemv(a.dir[0], a.dir[1], a.dir[2], a.dir[3], a.copy_bytes))
    elif a.pmc:
        print(pmc(a.dir, a.kernel, a.last))
    elif a.traffic:
        print(traffic(a.dir[0], a.dir[1], a.kernel, a.last, a.copy_bytes, a.config))
    else:
        print(summarise(a.dir[0], a.kernel, a.last, skip_last=a.skip_last, by_grid=a.by_grid))


if __name__ == "__main__":
    sys.exit(main())
