"""Text summaries of rocprofv3 CSV output for the attention kernels.

    python -m attentionfuse_amd.rocprof_summary stats DIR [--match S ...] [--by-grid]
    python -m attentionfuse_amd.rocprof_summary pmc DIR [DIR ...] [--match S ...] [--by-grid]
    python -m attentionfuse_amd.rocprof_summary traffic --fetch DIR --write DIR \
        --copy-fetch DIR --copy-write DIR --copy-bytes N [--match S ...] [--by-grid]

``stats`` reads ``*_kernel_stats.csv`` (``rocprofv3 --kernel-trace --stats
-f csv``); ``pmc`` reads ``*_counter_collection.csv`` (``rocprofv3 --pmc ...
-f csv``) and averages each counter per dispatch for every kernel whose name
contains one of the ``--match`` strings; ``traffic`` turns FETCH_SIZE and
WRITE_SIZE (KiB per dispatch) into HBM bytes per launch, scaled by what the
same counters read for a plain copy of ``--copy-bytes`` bytes read and
written, and prints one ``TRAFFIC <kernel> ...`` line per kernel.

``--by-grid`` keys every figure on (kernel, grid size) instead of the kernel
name alone, so one kernel launched on two workloads (the decode split kernel
at a 32k cache and at a short one) is reported as two rows; ``stats`` then
reads the per-dispatch ``*_kernel_trace.csv`` instead of the stats file.

Derived figures printed by ``pmc`` (when the counters are present):
GRBM_GUI_ACTIVE is summed over the 8 XCDs, so cycles = GRBM_GUI_ACTIVE / 8;
SQ_VALU_MFMA_BUSY_CYCLES is summed over the 1024 SIMDs (256 CUs x 4), so
the MFMA-busy fraction is busy / (cycles * 1024); the clock is cycles /
kernel duration.
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import os
import re
import sys


def _short(name: str) -> str:
    name = re.sub(r"^void ", "", name)
    return re.sub(r"\(.*\)$", "", name)


def _rows(dirs, suffix):
    for d in dirs:
        for f in sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True)):
            with open(f, newline="") as fh:
                yield from csv.DictReader(fh)


def _matches(name, match):
    return not match or any(m in name for m in match)


def _grid(r):
    if "Grid_Size" in r:
        return r["Grid_Size"]
    return "x".join(r[f"Grid_Size_{a}"] for a in "XYZ")


def _key(name, r, by_grid):
    k = _short(name)
    return f"{k} grid={_grid(r)}" if by_grid else k


def _trace_stats(dirs, match):
    durs = collections.defaultdict(list)
    for r in _rows(dirs, "_kernel_trace.csv"):
        if _matches(r["Kernel_Name"], match):
            durs[_key(r["Kernel_Name"], r, True)].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    total = sum(sum(v) for v in durs.values()) or 1
    out = [f"{'kernel':92s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s} {'total_%':>8s}"]
    for k, v in sorted(durs.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"{k[:92]:92s} {len(v):6d} {sum(v) / len(v) / 1e3:10.3f} {min(v) / 1e3:10.3f} "
                   f"{max(v) / 1e3:10.3f} {100.0 * sum(v) / total:8.2f}")
    return out


def stats(dirs, match, by_grid=False):
    if by_grid:
        return _trace_stats(dirs, match)
    out = []
    hdr = f"{'kernel':70s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s} {'total_%':>8s}"
    out.append(hdr)
    for r in _rows(dirs, "_kernel_stats.csv"):
        if not _matches(r["Name"], match):
            continue
        out.append(f"{_short(r['Name'])[:70]:70s} {int(r['Calls']):6d} "
                   f"{float(r['AverageNs']) / 1e3:10.3f} {float(r['MinNs']) / 1e3:10.3f} "
                   f"{float(r['MaxNs']) / 1e3:10.3f} {float(r['Percentage']):8.2f}")
    return out


def _pmc_means(dirs, match, by_grid=False):
    vals = collections.defaultdict(lambda: collections.defaultdict(list))
    durs = collections.defaultdict(dict)
    for r in _rows(dirs, "_counter_collection.csv"):
        name = r["Kernel_Name"]
        if not _matches(name, match):
            continue
        k = _key(name, r, by_grid)
        vals[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
        durs[k][r["Dispatch_Id"]] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    means = {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in vals.items()}
    counts = {k: {c: len(v) for c, v in cs.items()} for k, cs in vals.items()}
    return means, counts, durs


def pmc(dirs, match, by_grid=False):
    means, counts, durs = _pmc_means(dirs, match, by_grid)
    out = []
    for k in sorted(means):
        m = means[k]
        out.append(f"kernel {k}")
        for c in sorted(m):
            out.append(f"  {c:32s} {m[c]:16.6g}   (mean of {counts[k][c]} dispatches)")
        if "GRBM_GUI_ACTIVE" in m and "SQ_VALU_MFMA_BUSY_CYCLES" in m:
            cyc = m["GRBM_GUI_ACTIVE"] / 8
            out.append(f"  -> cycles {cyc:.0f}; MFMA busy fraction {m['SQ_VALU_MFMA_BUSY_CYCLES'] / (cyc * 1024):.3f}")
            if durs[k]:
                ns = sum(durs[k].values()) / len(durs[k])
                out.append(f"  -> mean dispatch duration under counters {ns / 1e3:.1f} us; "
                           f"clock {cyc / ns:.2f} GHz")
    return out


def traffic(fetch, write, copy_fetch, copy_write, copy_bytes, match, by_grid=False):
    f_means, _, _ = _pmc_means([fetch], match, by_grid)
    w_means, _, _ = _pmc_means([write], match, by_grid)
    cf, _, _ = _pmc_means([copy_fetch], ["neg"])
    cw, _, _ = _pmc_means([copy_write], ["neg"])
    if not cf or not cw:
        raise SystemExit("no copy-kernel dispatches in the calibration runs")
    cfk = max(cf.values(), key=lambda m: m.get("FETCH_SIZE", 0))["FETCH_SIZE"]
    cwk = max(cw.values(), key=lambda m: m.get("WRITE_SIZE", 0))["WRITE_SIZE"]
    sf = copy_bytes / (cfk * 1024.0)
    sw = copy_bytes / (cwk * 1024.0)
    out = [f"copy calibration: {copy_bytes} B read -> FETCH_SIZE {cfk:.6g} KiB (factor {sf:.4f}); "
           f"{copy_bytes} B written -> WRITE_SIZE {cwk:.6g} KiB (factor {sw:.4f})"]
    for k in sorted(set(f_means) & set(w_means)):
        fb = f_means[k].get("FETCH_SIZE", 0.0) * 1024.0 * sf
        wb = w_means[k].get("WRITE_SIZE", 0.0) * 1024.0 * sw
        out.append(f"TRAFFIC {k} fetch_bytes={fb:.0f} write_bytes={wb:.0f} total_bytes={fb + wb:.0f}")
    return out


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("stats")
    a.add_argument("dirs", nargs="+")
    a.add_argument("--match", nargs="*", default=[])
    a.add_argument("--by-grid", action="store_true")
    b = sub.add_parser("pmc")
    b.add_argument("dirs", nargs="+")
    b.add_argument("--match", nargs="*", default=[])
    b.add_argument("--by-grid", action="store_true")
    c = sub.add_parser("traffic")
    for n in ("fetch", "write", "copy-fetch", "copy-write"):
        c.add_argument("--" + n, required=True)
    c.add_argument("--copy-bytes", type=int, required=True)
    c.add_argument("--match", nargs="*", default=[])
    c.add_argument("--by-grid", action="store_true")
    args = ap.parse_args(argv)
    if args.cmd == "stats":
        lines = stats(args.dirs, args.match, args.by_grid)
    elif args.cmd == "pmc":
        lines = pmc(args.dirs, args.match, args.by_grid)
    else:
        lines = traffic(args.fetch, args.write, args.copy_fetch, args.copy_write,
                        args.copy_bytes, args.match, args.by_grid)
    sys.stdout.write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main()
