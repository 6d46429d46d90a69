"""Counter helpers for rocprofv3 --pmc runs.

``python -m trident_amd.profiling copy --mib 1024 --reps 3`` runs a plain device-to-device
copy of a known size; the FETCH_SIZE / WRITE_SIZE that rocprofv3 reports for that copy kernel,
divided into the bytes actually moved, gives the scale factor applied to the same counters
read on the scan kernel.

``python -m trident_amd.profiling summarize DIR --kernels REGEX [--out FILE]`` reduces the
``*counter_collection.csv`` of a rocprofv3 output directory to one record per kernel: the
number of dispatches, their mean duration and, per counter, the median over dispatches of the
per-dispatch value (rows of one dispatch and counter are summed).
"""
import argparse
import csv
import glob
import json
import os
import re
import statistics
import sys


def copy_probe(mib: int, reps: int) -> None:
    import torch
    n = mib * (1 << 20) // 4
    src = torch.arange(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copy_probe: {reps} copies of {mib} MiB ({n * 4} bytes read and written each)", flush=True)


def summarize(directory: str, kernels: str = "", out: str = "") -> dict:
    pat = re.compile(kernels) if kernels else None
    per = {}  # kernel -> {"t": {dispatch: ns}, "c": {counter: {dispatch: value}}}
    for path in sorted(glob.glob(os.path.join(directory, "*counter_collection.csv"))):
        with open(path, newline="") as f:
            for row in csv.DictReader(f):
                name = row["Kernel_Name"]
                if pat and not pat.search(name):
                    continue
                k = per.setdefault(name, {"t": {}, "c": {}})
                d = row["Dispatch_Id"]
                k["t"][d] = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
                c = k["c"].setdefault(row["Counter_Name"], {})
                c[d] = c.get(d, 0.0) + float(row["Counter_Value"])
    res = {}
    for name, k in per.items():
        res[name] = {"dispatches": len(k["t"]),
                     "avg_ms": statistics.mean(k["t"].values()) / 1e6 if k["t"] else None,
                     "median_per_dispatch": {c: statistics.median(v.values()) for c, v in sorted(k["c"].items())}}
    text = json.dumps(res, indent=1)
    if out:
        with open(out, "w") as f:
            f.write(text + "\n")
    print(text, flush=True)
    return res


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("copy")
    c.add_argument("--mib", type=int, default=1024)
    c.add_argument("--reps", type=int, default=3)
    m = sub.add_parser("summarize")
    m.add_argument("directory")
    m.add_argument("--kernels", default="")
    m.add_argument("--out", default="")
    a = ap.parse_args(argv)
    if a.cmd == "copy":
        copy_probe(a.mib, a.reps)
    elif a.cmd == "summarize":
        summarize(a.directory, a.kernels, a.out)


if __name__ == "__main__":
    main(sys.argv[1:])
