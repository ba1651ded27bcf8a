"""Condense rocprofv3 CSV output into the short text summaries kept under profiles/.

Usage (after the rocprofv3 runs listed in each summary's header)::

    python -m flashrnn_amd.rocprof_summary --workload NAME --cmd "..." \
        --kernel-trace DIR [--fetch DIR --write DIR --copy-fetch DIR --copy-write DIR --copy-mib M]
        [--sq DIR --active-cus C] --out profiles/

The kernel-trace summary lists per-kernel call counts and durations. The
traffic summary gives each kernel's FETCH_SIZE / WRITE_SIZE per dispatch
(KiB, as the counters read) and the bytes they stand for, after scaling each
counter by what it reads for a plain device copy of known size. The SQ
summary gives MFMA busy cycles and FLOP, the MFMA busy fraction of the CUs the
recurrence occupies, and LDS bank conflicts.
"""

from __future__ import annotations

import argparse
import collections
import csv
import glob
import os


def _one(d, pattern):
    files = sorted(glob.glob(os.path.join(d, "**", pattern), recursive=True))
    if not files:
        raise SystemExit(f"no {pattern} under {d}")
    return files[0]


def short(name: str) -> str:
    name = name.replace("(frnn::FwdArgs)", "").replace("(frnn::BwdArgs)", "").replace("(frnn::GemmArgs)", "")
    return name[5:] if name.startswith("void ") else name


def kernel_stats(d):
    rows = list(csv.DictReader(open(_one(d, "*kernel_stats.csv"))))
    return [(short(r["Name"]), int(r["Calls"]), float(r["AverageNs"]), float(r["MinNs"]), float(r["MaxNs"]),
             float(r["Percentage"])) for r in rows]


def counter(d, name):
    agg = collections.defaultdict(list)
    for r in csv.DictReader(open(_one(d, "*counter_collection.csv"))):
        if r["Counter_Name"] == name:
            agg[short(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in agg.items()}


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", required=True)
    ap.add_argument("--cmd", required=True, help="the rocprofv3 command lines that produced the CSVs")
    ap.add_argument("--kernel-trace", required=True)
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--copy-fetch")
    ap.add_argument("--copy-write")
    ap.add_argument("--copy-mib", type=int, default=512)
    ap.add_argument("--sq", help="counter CSVs of one pass over SQ_VALU_MFMA_BUSY_CYCLES, "
                    "SQ_INSTS_VALU_MFMA_MOPS_BF16, SQ_LDS_BANK_CONFLICT, SQ_LDS_IDX_ACTIVE, SQ_INSTS_LDS, "
                    "SQ_BUSY_CU_CYCLES, GRBM_GUI_ACTIVE")
    ap.add_argument("--active-cus", type=int, default=48, help="CUs the persistent kernels occupy")
    ap.add_argument("--clock-mhz", type=float, default=2400.0)
    ap.add_argument("--out", default="profiles")
    a = ap.parse_args(argv)

    stats = kernel_stats(a.kernel_trace)
    lines = [f"# rocprofv3 kernel trace: {a.workload}", "", "Command:", "", *[f"    {c}" for c in a.cmd.split(";;")], "",
             f"{'kernel':60s} {'calls':>6s} {'avg_us':>10s} {'min_us':>10s} {'max_us':>10s} {'pct':>6s}"]
    for n, c, avg, mn, mx, pct in stats:
        lines.append(f"{n[:60]:60s} {c:6d} {avg / 1e3:10.1f} {mn / 1e3:10.1f} {mx / 1e3:10.1f} {pct:6.2f}")
    os.makedirs(a.out, exist_ok=True)
    p1 = os.path.join(a.out, f"kernel_trace_{a.workload}.txt")
    open(p1, "w").write("\n".join(lines) + "\n")
    print(p1)

    if a.fetch and a.write and a.copy_fetch and a.copy_write:
        kib = a.copy_mib * 1024
        cf = max(counter(a.copy_fetch, "FETCH_SIZE").items(), key=lambda kv: kv[1])
        cw = max(counter(a.copy_write, "WRITE_SIZE").items(), key=lambda kv: kv[1])
        ff, fw = kib / cf[1], kib / cw[1]
        fetch, write = counter(a.fetch, "FETCH_SIZE"), counter(a.write, "WRITE_SIZE")
        lines = [f"# HBM traffic per dispatch: {a.workload}", "", "Command:", "",
                 *[f"    {c}" for c in a.cmd.split(";;")], "",
                 f"Calibration: a {a.copy_mib} MiB device copy ({cf[0]}) reads FETCH_SIZE {cf[1]:.1f} KiB and "
                 f"WRITE_SIZE {cw[1]:.1f} KiB per dispatch; scale factors fetch {ff:.4f}, write {fw:.4f}.", "",
                 f"{'kernel':48s} {'FETCH_KiB':>12s} {'WRITE_KiB':>12s} {'read_MB':>10s} {'write_MB':>10s} "
                 f"{'traffic_bytes':>14s}"]
        for n in fetch:
            if n not in write:
                continue
            rb, wb = fetch[n] * ff * 1024, write[n] * fw * 1024
            lines.append(f"{n[:48]:48s} {fetch[n]:12.1f} {write[n]:12.1f} {rb / 1e6:10.2f} {wb / 1e6:10.2f} "
                         f"{rb + wb:14.0f}")
        p2 = os.path.join(a.out, f"hbm_traffic_{a.workload}.txt")
        open(p2, "w").write("\n".join(lines) + "\n")
        print(p2)

    if a.sq:
        names = ["SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_LDS_BANK_CONFLICT",
                 "SQ_LDS_IDX_ACTIVE", "SQ_INSTS_LDS", "SQ_BUSY_CU_CYCLES", "GRBM_GUI_ACTIVE"]
        c = {n: counter(a.sq, n) for n in names}
        dur = {n: avg for n, _, avg, *_ in stats}
        lines = [f"# SQ counters per dispatch: {a.workload}", "", "Command:", "",
                 *[f"    {x}" for x in a.cmd.split(";;")], "",
                 "Columns: MFMA busy cycles (summed over SIMDs) and BF16 MFMA FLOP (MOPS x 512); MFMA busy",
                 f"fraction of the SIMDs of the {a.active_cus} CUs the recurrence occupies over the kernel's traced",
                 f"duration at {a.clock_mhz:.0f} MHz (whole chip: x {a.active_cus}/256); LDS bank-conflict cycles,",
                 "and conflict cycles per conflict-free LDS cycle (SQ_LDS_BANK_CONFLICT / (SQ_LDS_IDX_ACTIVE -",
                 "SQ_LDS_BANK_CONFLICT)); LDS instructions.", "",
                 f"{'kernel':40s} {'mfma_busy':>12s} {'bf16_GFLOP':>11s} {'busy_frac':>9s} {'lds_conflict':>13s} "
                 f"{'confl_ratio':>11s} {'lds_insts':>11s}"]
        for n in c["SQ_VALU_MFMA_BUSY_CYCLES"]:
            busy = c["SQ_VALU_MFMA_BUSY_CYCLES"][n]
            flop = c["SQ_INSTS_VALU_MFMA_MOPS_BF16"].get(n, 0.0) * 512
            conf = c["SQ_LDS_BANK_CONFLICT"].get(n, 0.0)
            act = c["SQ_LDS_IDX_ACTIVE"].get(n, 0.0)
            ratio = conf / (act - conf) if act > conf else 0.0
            d = dur.get(n)
            frac = busy / (d * 1e-3 * a.clock_mhz * 4 * a.active_cus) if d else float("nan")
            lines.append(f"{n[:40]:40s} {busy:12.0f} {flop / 1e9:11.3f} {frac:9.4f} {conf:13.0f} {ratio:11.4f} "
                         f"{c['SQ_INSTS_LDS'].get(n, 0.0):11.0f}")
        p3 = os.path.join(a.out, f"sq_counters_{a.workload}.txt")
        open(p3, "w").write("\n".join(lines) + "\n")
        print(p3)


if __name__ == "__main__":
    main()
