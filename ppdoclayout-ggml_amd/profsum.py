"""Summaries of rocprofv3 output for profiles/ (run on the CSVs a GPU run wrote).

  python profsum.py stats   <kernel_stats.csv>                 > table (markdown)
  python profsum.py traffic <fetch_dir> <write_dir> <copy_MiB> > per-kernel HBM bytes (JSON)
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


def per_dispatch(directory, counter):
    """{dispatch_id: (kernel, value summed over instances)}"""
    acc = {}
    for f in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] != counter:
                continue
            d = r["Dispatch_Id"]
            k, v = acc.get(d, (r["Kernel_Name"], 0.0))
            acc[d] = (k, v + float(r["Counter_Value"]))
    return acc


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
    elif len(sys.argv) >= 6 and sys.argv[1] == "dispatches":
        print(dispatches(sys.argv[2], sys.argv[3], int(sys.argv[4]), int(sys.argv[5])))
    else:
        sys.exit(__doc__)
