#!/usr/bin/env python3
"""Summaries of rocprofv3 counter runs of bench.py workloads, as bench.py reads them.

Each --entry names a workload and the output directories of its counter runs (rocprofv3
--pmc ... --output-format csv -d DIR -o run); counters are matched to this library's kernels
(names starting with "w4a16::").  HBM bytes per launch come from FETCH_SIZE and WRITE_SIZE (KiB
per dispatch), scaled by what the same counters read for the copy calibration workload
(bench.py --workload copy: 64 MiB read and 64 MiB written per launch).  A run that also holds
SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE gives the matrix-core busy fraction (over 4 SIMDs
x cu_count CUs) and the shader clock (GRBM_GUI_ACTIVE per XCD over the dispatch duration).

    python w4a16-gemm_amd/pmc_summary.py --copy gpurun_out/cpyF gpurun_out/cpyW \\
        --entry decode=gpurun_out/decF,gpurun_out/decW --source profiles/X.md --out profiles/traffic.json
"""
from __future__ import annotations

import argparse
import collections
import csv
import json
import os
import statistics
import sys

COPY_BYTES = 64 * 2**20          # bench.py --workload copy: bytes read (and written) per launch
XCDS = 8


def kernel_name(raw: str) -> str:
    """The kernel's name without its argument list (demangled with c++filt when rocprofv3 left it
    mangled)."""
    if raw.startswith("_Z"):
        # binutils' c++filt does not know _Float16 (DF16_): demangle it as decltype(nullptr) (Dn),
        # which cannot occur in these kernels' names, and put the type back.
        import subprocess
        try:
            out = subprocess.run(["c++filt", raw.replace("DF16_", "Dn")], capture_output=True, text=True,
                                 check=True).stdout.strip()
        except (OSError, subprocess.CalledProcessError):
            return raw
        raw = out.replace("decltype(nullptr)", "_Float16")
    raw = raw.replace("void ", "", 1).strip() if raw.startswith("void ") else raw.strip()
    if raw.endswith(")"):                              # drop the argument list: the outermost (...) at the end
        depth = 0
        for i in range(len(raw) - 1, -1, -1):
            depth += {")": 1, "(": -1}.get(raw[i], 0)
            if depth == 0:
                return raw[:i].strip()
    return raw


def read_runs(dirs):
    """{kernel: {counter: [values]}} and {kernel: [durations ns]} over the runs' dispatches."""
    vals = collections.defaultdict(lambda: collections.defaultdict(list))
    durs = collections.defaultdict(list)
    for d in dirs:
        path = os.path.join(d, "run_counter_collection.csv")
        seen = set()
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                name = kernel_name(r["Kernel_Name"])
                vals[name][r["Counter_Name"]].append(float(r["Counter_Value"]))
                key = (name, r["Dispatch_Id"])
                if key not in seen:
                    seen.add(key)
                    durs[name].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    return vals, durs


def median(xs):
    return statistics.median(xs) if xs else None


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--copy", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"), required=True)
    ap.add_argument("--entry", action="append", default=[], help="kind=DIR[,DIR...] (repeatable)")
    ap.add_argument("--cus", type=int, default=256)
    ap.add_argument("--source", required=True, help="the summary file the figures are quoted in")
    ap.add_argument("--out", required=True, help="JSON file to update (kinds not given are kept)")
    a = ap.parse_args(argv)

    cf, _ = read_runs([a.copy[0]])
    cw, _ = read_runs([a.copy[1]])
    fetch_copy = median([v for k in cf for v in cf[k].get("FETCH_SIZE", [])])
    write_copy = median([v for k in cw for v in cw[k].get("WRITE_SIZE", [])])
    fscale = COPY_BYTES / 1024 / fetch_copy
    wscale = COPY_BYTES / 1024 / write_copy
    print(f"copy calibration: FETCH_SIZE {fetch_copy:.0f} KiB -> x{fscale:.4f}, WRITE_SIZE {write_copy:.0f} KiB -> x{wscale:.4f}")

    try:
        with open(a.out) as f:
            doc = json.load(f)
    except (OSError, ValueError):
        doc = {}
    doc = {k: v for k, v in doc.items() if isinstance(v, dict)}
    for spec in a.entry:
        kind, dirs = spec.split("=", 1)
        vals, durs = read_runs(dirs.split(","))
        kernels = sorted(k for k in vals if k.startswith("w4a16::"))
        ent = {"kernels": kernels, "source": a.source, "per_kernel": {}}
        traffic = []
        for k in kernels:
            c = vals[k]
            row = {}
            if "FETCH_SIZE" in c and "WRITE_SIZE" in c:
                row["fetch_kib"] = median(c["FETCH_SIZE"])
                row["write_kib"] = median(c["WRITE_SIZE"])
                row["hbm_bytes"] = round((row["fetch_kib"] * fscale + row["write_kib"] * wscale) * 1024)
                traffic.append(row["hbm_bytes"])
            if "SQ_VALU_MFMA_BUSY_CYCLES" in c and "GRBM_GUI_ACTIVE" in c:
                cyc = median(c["GRBM_GUI_ACTIVE"]) / XCDS
                row["mfma_busy_frac"] = round(median(c["SQ_VALU_MFMA_BUSY_CYCLES"]) / (cyc * 4 * a.cus), 4)
                row["clock_ghz"] = round(cyc / median(durs[k]), 3)
            row["duration_us"] = round(median(durs[k]) / 1e3, 2)
            ent["per_kernel"][k] = row
            print(kind, k, row)
        if traffic:
            ent["traffic"] = round(statistics.mean(traffic))
        busy = [r["mfma_busy_frac"] for r in ent["per_kernel"].values() if "mfma_busy_frac" in r]
        if busy:
            ent["mfma_busy_frac"] = round(statistics.mean(busy), 4)
            ent["clock_ghz"] = round(statistics.mean(r["clock_ghz"] for r in ent["per_kernel"].values()
                                                     if "clock_ghz" in r), 3)
        ent["fetch_size_scale"], ent["write_size_scale"] = round(fscale, 4), round(wscale, 4)
        doc[kind] = ent
    with open(a.out, "w") as f:
        json.dump(doc, f, indent=1, sort_keys=True)
        f.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
