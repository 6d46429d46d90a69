"""Counter calibration helper for rocprofv3 --pmc runs.

``python -m trident_amd.profiling copy --mib 1024 --reps 3`` runs a plain device-to-device
copy of a known size; the FETCH_SIZE / WRITE_SIZE that rocprofv3 reports for that copy kernel,
divided into the bytes actually moved, gives the scale factor applied to the same counters
read on the scan kernel.
"""
import argparse
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


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("copy")
    c.add_argument("--mib", type=int, default=1024)
    c.add_argument("--reps", type=int, default=3)
    a = ap.parse_args(argv)
    if a.cmd == "copy":
        copy_probe(a.mib, a.reps)


if __name__ == "__main__":
    main(sys.argv[1:])
