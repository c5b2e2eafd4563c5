"""Summaries of rocprofv3 output for profiles/ (run on the CSVs a GPU run wrote).

  python profsum.py stats   <kernel_stats.csv>                 > table (markdown)
  python profsum.py traffic <fetch_dir> <write_dir> <copy_MiB> > per-kernel HBM bytes (JSON)
  python profsum.py mfma <pmc_dir>                         > per-kernel MFMA counters (markdown)
  python profsum.py dispatches <fetch_dir> <write_dir> <copy_MiB> <count>
                                                          > the first <count> library dispatches in
                                                            launch order with their HBM bytes (markdown)

stats: one row per kernel symbol: calls, mean and total duration.

traffic: FETCH_SIZE and WRITE_SIZE (KiB per dispatch, from two separate
`rocprofv3 --pmc` runs) averaged per kernel symbol, each scaled by what the
same counter reads for a plain elementwise copy of `copy_MiB` MiB that ran in
the same process (bench.py --calib-copy-mib): the copy reads and writes exactly
that many bytes, so factor = true bytes / counter bytes.  The copy is the
dispatch with the largest counter value among kernels that are not this
library's.
"""
import csv
import glob
import json
import os
import re
import sys
from collections import defaultdict


def short(name):
    n = name.replace("ppdl::(anonymous namespace)::", "").replace("void ", "")
    return re.sub(r"\(.*$", "", n).strip()


def stats(path):
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    out = ["| kernel | calls | mean us | total us |", "|---|---|---|---|"]
    for r in rows:
        out.append("| `%s` | %s | %.2f | %.1f |" % (short(r["Name"]), r["Calls"], float(r["AverageNs"]) / 1e3,
                                                    float(r["TotalDurationNs"]) / 1e3))
    return "\n".join(out)


def per_dispatch(directory, counter, reduce=sum):
    """{dispatch_id: (kernel, value reduced over instances)}"""
    vals = {}
    for f in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] != counter:
                continue
            vals.setdefault(r["Dispatch_Id"], (r["Kernel_Name"], []))[1].append(float(r["Counter_Value"]))
    return {d: (k, reduce(v)) for d, (k, v) in vals.items()}


def traffic(fetch_dir, write_dir, copy_mib):
    copy_bytes = copy_mib * (1 << 20)
    res = {}
    factors = {}
    for counter, directory in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        disp = per_dispatch(directory, counter)
        foreign = [v for (k, v) in disp.values() if "ppdl::" not in k]
        if not foreign:
            raise SystemExit("no calibration copy found in " + directory)
        fac = copy_bytes / (max(foreign) * 1024.0)  # counters are KiB
        factors[counter] = fac
        by = defaultdict(list)
        for k, v in disp.values():
            if "ppdl::" in k:
                by[short(k)].append(v * 1024.0 * fac)
        for k, vals in by.items():
            res.setdefault(k, {})[counter] = sum(vals) / len(vals)
            res[k]["dispatches"] = len(vals)
    kernels = {}
    for k, v in res.items():
        f, w = v.get("FETCH_SIZE"), v.get("WRITE_SIZE")
        kernels[k] = {"fetch_bytes": round(f) if f is not None else None,
                      "write_bytes": round(w) if w is not None else None,
                      "bytes": round(f + w) if f is not None and w is not None else None,
                      "dispatches": v["dispatches"]}
    return {"calibration": {"copy_MiB": copy_mib, "FETCH_SIZE_factor": round(factors["FETCH_SIZE"], 4),
                            "WRITE_SIZE_factor": round(factors["WRITE_SIZE"], 4)},
            "kernels": kernels}


def mfma(directory):
    """Per kernel: FP32 MFMA FLOP per dispatch (SQ_INSTS_VALU_MFMA_MOPS_F32 x 512),
    XF32 MFMA instructions (SQ_INSTS_VALU_MFMA_XF32), MFMA busy share of SIMD
    cycles and, with the kernel trace of the same run, the counted FLOP over the
    dispatch duration.  The busy share is SQ_VALU_MFMA_BUSY_CYCLES (summed over
    SIMDs) / (SIMDs x active cycles), where GRBM_GUI_ACTIVE arrives summed over
    the XCDs and is divided by their count (Num_Xcc of the agent info)."""
    names = ("SQ_INSTS_VALU_MFMA_MOPS_F32", "SQ_INSTS_VALU_MFMA_XF32", "SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE")
    per = {n: per_dispatch(directory, n) for n in names}
    dur = {}
    for f in glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            dur[r["Dispatch_Id"]] = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
    simds, xcc = 1024, 8
    for f in glob.glob(os.path.join(directory, "**", "*agent_info.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if r.get("Name", "").startswith("gfx"):
                simds, xcc = int(r["Simd_Count"]), int(r["Num_Xcc"])
    agg = defaultdict(lambda: [0, 0.0, 0.0, 0.0, 0.0, 0.0])  # n, flop, xf32, busy, active, ns
    for d, (k, mops) in per[names[0]].items():
        if "ppdl::" not in k:
            continue
        a = agg[short(k)]
        a[0] += 1
        a[1] += mops * 512.0
        a[2] += per[names[1]].get(d, (k, 0.0))[1]
        a[3] += per[names[2]].get(d, (k, 0.0))[1]
        a[4] += per[names[3]].get(d, (k, 0.0))[1]
        a[5] += dur.get(d, 0.0)
    out = ["| kernel | dispatches | MFMA FP32 GFLOP per dispatch | XF32 MFMA instr | MFMA busy % | us per dispatch "
           "(counter run) | counted TF/s |", "|---|---|---|---|---|---|---|"]
    for k, (n, fl, xf, busy, act, ns) in sorted(agg.items(), key=lambda kv: -kv[1][1]):
        if fl <= 0:
            continue
        util = 100.0 * busy / (act / xcc * simds) if act > 0 else 0.0
        us = ns / n / 1e3 if ns > 0 else 0.0
        tf = fl / ns / 1e3 if ns > 0 else 0.0
        out.append("| `%s` | %d | %.4f | %d | %.1f | %.2f | %.1f |" % (k, n, fl / n / 1e9, xf, util, us, tf))
    return "\n".join(out)


def dispatches(fetch_dir, write_dir, copy_mib, count):
    """First `count` library dispatches (launch order) with scaled FETCH/WRITE MB."""
    copy_bytes = copy_mib * (1 << 20)
    cols = {}
    for counter, directory in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        disp = per_dispatch(directory, counter)
        foreign = [v for (k, v) in disp.values() if "ppdl::" not in k]
        if not foreign:
            raise SystemExit("no calibration copy found in " + directory)
        fac = copy_bytes / (max(foreign) * 1024.0)
        mine = sorted(((int(d), k, v) for d, (k, v) in disp.items() if "ppdl::" in k))[:count]
        cols[counter] = [(short(k), v * 1024.0 * fac / 1e6) for (_, k, v) in mine]
    out = ["| # | kernel | FETCH MB | WRITE MB |", "|---|---|---|---|"]
    for i, ((k, f), (k2, w)) in enumerate(zip(cols["FETCH_SIZE"], cols["WRITE_SIZE"])):
        out.append("| %d | `%s` | %.2f | %.2f |" % (i, k if k == k2 else k + " / " + k2, f, w))
    return "\n".join(out)


if __name__ == "__main__":
    if len(sys.argv) >= 3 and sys.argv[1] == "stats":
        print(stats(sys.argv[2]))
    elif len(sys.argv) >= 5 and sys.argv[1] == "traffic":
        print(json.dumps(traffic(sys.argv[2], sys.argv[3], int(sys.argv[4])), indent=1, sort_keys=True))
    elif len(sys.argv) >= 3 and sys.argv[1] == "mfma":
        print(mfma(sys.argv[2]))
    elif len(sys.argv) >= 6 and sys.argv[1] == "dispatches":
        print(dispatches(sys.argv[2], sys.argv[3], int(sys.argv[4]), int(sys.argv[5])))
    else:
        sys.exit(__doc__)
