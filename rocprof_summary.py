"""Summarises rocprofv3 CSV output of ``bench.py`` into the text kept under ``profiles/``.

    python rocprof_summary.py --trace DIR --fetch DIR \\
        --write DIR [--mfma DIR] --kv-bytes N --command "..." --out profiles/FILE.txt

Inputs are the directories rocprofv3 wrote with ``--output-format csv``:
``--kernel-trace --stats`` (``*_kernel_stats.csv``), ``--pmc FETCH_SIZE``,
``--pmc WRITE_SIZE`` and optionally ``--pmc SQ_VALU_MFMA_BUSY_CYCLES
GRBM_GUI_ACTIVE ...`` (``*_counter_collection.csv``).

Byte counters are calibrated with the plain 1 GiB device copy that
``bench.py --copy-probe-mib 1024`` runs first: the copy reads and writes
exactly 1 GiB, so ``scale = 2**30 / (counter KiB * 1024)`` for each counter.
"""

from __future__ import annotations

import argparse
import collections
import csv
import glob
import os
from pathlib import Path

COPY_BYTES = 1 << 30


def _one(pattern):
    hits = glob.glob(pattern, recursive=True)
    if not hits:
        raise SystemExit(f"no file matches {pattern}")
    return hits[0]


def _short(name):
    name = name.replace("void ", "").replace("sqa::", "").replace("(anonymous namespace)::", "")
    return name.split("(")[0]


def kernel_stats(trace_dir):
    rows = list(csv.DictReader(open(_one(os.path.join(trace_dir, "**", "*kernel_stats.csv")))))
    return {_short(r["Name"]): (int(r["Calls"]), float(r["AverageNs"]) / 1e3,
                               float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3)
            for r in rows if "sqa" in r["Name"]}


def last_dispatches_us(trace_dir, n):
    """Mean duration (us) of each kernel's last ``n`` dispatches: the bench's timed steps
    (the warmup and clock-ramp calls come first)."""
    hits = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not hits or n <= 0:
        return {}
    per = collections.defaultdict(list)
    for r in csv.DictReader(open(hits[0])):
        if "sqa" in r["Kernel_Name"]:
            per[_short(r["Kernel_Name"])].append(
                (int(r["Start_Timestamp"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    out = {}
    for name, d in per.items():
        d.sort()
        tail = [dur for _, dur in d[-n:]]
        out[name] = sum(tail) / len(tail) / 1e3
    return out


def counters(pmc_dir):
    rows = list(csv.DictReader(open(_one(os.path.join(pmc_dir, "**", "*counter_collection.csv")))))
    per = collections.defaultdict(list)
    copy = []
    for r in rows:
        val = float(r["Counter_Value"])
        if "sqa" in r["Kernel_Name"]:
            per[(_short(r["Kernel_Name"]), r["Counter_Name"])].append(val)
        elif "copyBuffer" in r["Kernel_Name"] and int(r["Grid_Size"]) >= 65536:
            copy.append((r["Counter_Name"], val))
    return per, copy


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--trace", required=True)
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--mfma")
    ap.add_argument("--kv-bytes", type=int, required=True, help="algorithmic KV bytes per call")
    ap.add_argument("--steps", type=int, default=20,
                    help="timed steps of the traced bench run (their dispatches come last)")
    ap.add_argument("--workload", required=True)
    ap.add_argument("--command", required=True, help="the command line that produced the CSVs")
    ap.add_argument("--out", required=True)
    args = ap.parse_args(argv)

    stats = kernel_stats(args.trace)
    timed = last_dispatches_us(args.trace, args.steps)
    fetch, fcopy = counters(args.fetch)
    write, wcopy = counters(args.write)
    fscale = COPY_BYTES / (1024 * sum(v for _, v in fcopy) / len(fcopy))
    wscale = COPY_BYTES / (1024 * sum(v for _, v in wcopy) / len(wcopy))
    lines = [f"# rocprofv3 summary: {args.workload}",
             f"# command: {args.command}",
             "# byte counters calibrated with a plain 1 GiB device copy (bench.py --copy-probe-mib 1024):",
             f"fetch_scale: {fscale:.4f}",
             f"write_scale: {wscale:.4f}",
             f"kv_bytes_algorithmic: {args.kv_bytes}",
             ""]
    lines.append("kernel | calls | avg_us | min_us | max_us | fetch_bytes | write_bytes | fetch/alg")
    partial_traffic = None
    for name, (calls, avg, mn, mx) in sorted(stats.items()):
        fb = fetch.get((name, "FETCH_SIZE"))
        wb = write.get((name, "WRITE_SIZE"))
        fbytes = sum(fb) / len(fb) * 1024 * fscale if fb else float("nan")
        wbytes = sum(wb) / len(wb) * 1024 * wscale if wb else float("nan")
        ratio = fbytes / args.kv_bytes
        lines.append(f"{name} | {calls} | {avg:.2f} | {mn:.2f} | {mx:.2f} | {fbytes:.4e} | "
                     f"{wbytes:.4e} | {ratio:.4f}")
        if name.startswith("sqa_partial"):
            partial_traffic = fbytes + wbytes
            lines.append(f"partial_kernel_avg_us: {avg:.2f}")
            lines.append(f"partial_kernel_kv_GBps: {args.kv_bytes / (avg * 1e-6) / 1e9:.1f}")
            if name in timed:
                t = timed[name]
                lines.append(f"partial_kernel_timed_steps_avg_us: {t:.2f} (last {args.steps} "
                             "dispatches = the bench's timed steps)")
                lines.append(f"partial_kernel_timed_steps_kv_GBps: "
                             f"{args.kv_bytes / (t * 1e-6) / 1e9:.1f}")
        if name.startswith("sqa_merge_kernel") and name in timed:
            lines.append(f"merge_kernel_timed_steps_avg_us: {timed[name]:.2f} (last "
                         f"{args.steps} dispatches)")
    if partial_traffic is not None:
        lines.append(f"traffic_bytes_per_launch: {partial_traffic:.0f}")
    if args.mfma:
        mf, _ = counters(args.mfma)
        for name in sorted({k[0] for k in mf}):
            busy = mf.get((name, "SQ_VALU_MFMA_BUSY_CYCLES"))
            gui = mf.get((name, "GRBM_GUI_ACTIVE"))
            if busy and gui:
                # GRBM_GUI_ACTIVE is summed over the 8 XCDs; per-XCD cycles = sum / 8.
                b = sum(busy) / len(busy)
                g = sum(gui) / len(gui) / 8
                lines.append(f"{name} mfma_busy_pct: {100.0 * b / (g * 1024):.2f} "
                             f"(SQ_VALU_MFMA_BUSY_CYCLES {b:.4e} over 1024 SIMDs x "
                             f"{g:.4e} GRBM_GUI_ACTIVE cycles per XCD)")
    Path(args.out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


if __name__ == "__main__":
    main()
