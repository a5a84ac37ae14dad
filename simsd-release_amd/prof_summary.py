#!/usr/bin/env python3
"""Summarise rocprofv3 CSV output into the short text kept under profiles/.

    python simsd-release_amd/prof_summary.py stats DIR [--match SUBSTR ...]
    python simsd-release_amd/prof_summary.py pmc DIR [--match SUBSTR ...]
        [--calib DIR --calib-match SUBSTR --calib-bytes N]
    python simsd-release_amd/prof_summary.py mfma DIR [--match SUBSTR ...] [--stats-dir DIR]

``stats`` reads ``*_kernel_stats.csv`` (from ``rocprofv3 --kernel-trace
--stats``) and prints calls / average / min / max per kernel plus the
call-weighted average over the matched kernels.

``pmc`` reads ``*_counter_collection.csv`` (from ``rocprofv3 --pmc ...``) and
prints the average value per dispatch of every counter for every matched
kernel.  With ``--calib`` the same counters from a run of a plain copy kernel
that moves a known number of bytes each way give a scale factor
(known bytes / counter bytes), applied to the matched kernels' figures: the
counters are in KiB, and the factor absorbs whatever the counter misses or
double-counts on this part.
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import re
import sys
from collections import defaultdict


def short_name(name: str) -> str:
    """Kernel name without 'void ', the namespace and the argument list."""
    name = name.strip().strip('"').replace("(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    depth, cut = 0, len(name)
    for i, ch in enumerate(name):   # the first '(' outside template brackets
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            cut = i
            break
    name = name[:cut]
    return re.sub(r"^simsd::", "", name)


def _rows(directory: str, suffix: str):
    paths = sorted(glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True))
    if not paths:
        sys.exit(f"no *{suffix} under {directory}")
    for p in paths:
        with open(p, newline="") as f:
            yield from csv.DictReader(f)


def _matches(name: str, subs) -> bool:
    return not subs or any(s in name for s in subs)


def stats(directory: str, subs) -> str:
    out = [f"{'kernel':<60} {'calls':>7} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'pct':>6}"]
    tot_calls, tot_ns = 0, 0.0
    for r in _rows(directory, "_kernel_stats.csv"):
        name = short_name(r["Name"])
        if not _matches(name, subs):
            continue
        calls, avg = int(r["Calls"]), float(r["AverageNs"])
        tot_calls += calls
        tot_ns += calls * avg
        out.append(f"{name[:60]:<60} {calls:>7} {avg / 1e3:>9.3f} {float(r['MinNs']) / 1e3:>9.3f} "
                   f"{float(r['MaxNs']) / 1e3:>9.3f} {float(r['Percentage']):>6.2f}")
    if tot_calls:
        out.append(f"{'matched, call-weighted':<60} {tot_calls:>7} {tot_ns / tot_calls / 1e3:>9.3f}")
    return "\n".join(out)


def _pmc_table(directory: str, subs):
    acc = defaultdict(lambda: defaultdict(list))   # kernel -> counter -> values
    for r in _rows(directory, "_counter_collection.csv"):
        name = short_name(r["Kernel_Name"])
        if _matches(name, subs):
            acc[name][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return acc


def pmc(directory: str, subs, calib=None, calib_subs=None, calib_bytes=0) -> str:
    acc = _pmc_table(directory, subs)
    scale = {}
    out = []
    if calib:
        cal = _pmc_table(calib, calib_subs)
        for kern, counters in cal.items():
            for cname, vals in counters.items():
                kib = sum(vals) / len(vals)
                scale[cname] = calib_bytes / (kib * 1024.0) if kib > 0 else float("nan")
                out.append(f"calibration {kern[:48]} {cname}: {kib:.1f} KiB/dispatch for "
                           f"{calib_bytes} B -> factor {scale[cname]:.4f}")
    out.append(f"{'kernel':<60} {'counter':<12} {'dispatches':>10} {'KiB/disp':>12} {'bytes/disp (scaled)':>20}")
    totals = defaultdict(lambda: [0, 0.0])
    for kern in sorted(acc):
        for cname, vals in sorted(acc[kern].items()):
            kib = sum(vals) / len(vals)
            scaled = kib * 1024.0 * scale.get(cname, 1.0)
            totals[cname][0] += len(vals)
            totals[cname][1] += scaled * len(vals)
            out.append(f"{kern[:60]:<60} {cname:<12} {len(vals):>10} {kib:>12.1f} {scaled:>20.0f}")
    for cname, (n, s) in sorted(totals.items()):
        out.append(f"{'matched, dispatch-weighted':<60} {cname:<12} {n:>10} {'':>12} {s / n:>20.0f}")
    return "\n".join(out)


def mfma(directory: str, subs, simds: int, stats_dir=None) -> str:
    """MFMA utilisation per kernel from a run with SQ_VALU_MFMA_BUSY_CYCLES,
    GRBM_GUI_ACTIVE and SQ_INSTS_VALU_MFMA_MOPS_BF16: busy MFMA cycles summed
    over the SIMDs / (GPU-active cycles x SIMDs), the rocprofv3 MfmaUtil
    formula; with a stats run of the same workload, also the achieved bf16
    MFMA rate (MOPS x 512 flops per dispatch / average kernel time)."""
    acc = _pmc_table(directory, subs)
    avg_ns = {}
    if stats_dir:
        for r in _rows(stats_dir, "_kernel_stats.csv"):
            avg_ns[short_name(r["Name"])] = float(r["AverageNs"])
    out = [f"{'kernel':<60} {'disp':>5} {'mfma_busy':>12} {'gui_active':>11} {'util_%':>7} {'mfma_flop':>13} "
           f"{'TFLOP/s':>8}"]
    for kern in sorted(acc):
        c = acc[kern]
        mean = lambda n: sum(c[n]) / len(c[n]) if c.get(n) else float("nan")
        busy, gui, mops = mean("SQ_VALU_MFMA_BUSY_CYCLES"), mean("GRBM_GUI_ACTIVE"), mean("SQ_INSTS_VALU_MFMA_MOPS_BF16")
        util = 100.0 * busy / (gui * simds) if gui > 0 else float("nan")
        flop = mops * 512.0
        rate = flop / avg_ns[kern] / 1e3 if kern in avg_ns and avg_ns[kern] > 0 else float("nan")
        n = len(c.get("GRBM_GUI_ACTIVE", []))
        out.append(f"{kern[:60]:<60} {n:>5} {busy:>12.0f} {gui:>11.0f} {util:>7.2f} {flop:>13.0f} {rate:>8.2f}")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("mode", choices=["stats", "pmc", "mfma"])
    ap.add_argument("dir")
    ap.add_argument("--match", nargs="*", default=[])
    ap.add_argument("--calib")
    ap.add_argument("--calib-match", nargs="*", default=[])
    ap.add_argument("--calib-bytes", type=int, default=0)
    ap.add_argument("--simds", type=int, default=1024, help="SIMDs on the device (256 CUs x 4 on MI355X)")
    ap.add_argument("--stats-dir", help="mfma: a --kernel-trace --stats run of the same workload")
    a = ap.parse_args()
    if a.mode == "stats":
        print(stats(a.dir, a.match))
    elif a.mode == "mfma":
        print(mfma(a.dir, a.match, a.simds, a.stats_dir))
    else:
        print(pmc(a.dir, a.match, a.calib, a.calib_match, a.calib_bytes))


if __name__ == "__main__":
    main()
