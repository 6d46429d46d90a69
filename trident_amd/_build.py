"""Builds libtrident_hip.so in-tree with hipcc for gfx950.

Each .hip source is compiled to an object in trident_amd/_build/ and linked into
trident_amd/libtrident_hip.so.  Flags:
  --offload-arch=gfx950                      MI355X only
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                             no packed FP32 (v_pk_*_f32) instructions in the
                                             device code.  hipcc hands the flag to both of its
                                             passes; the x86 host pass does not know the feature
                                             and prints "'-packed-fp32-ops' is not a recognized
                                             feature for this target (ignoring feature)", which
                                             this script drops (hipcc cannot forward -Xclang
                                             options to the device pass alone).  The gfx950
                                             pass honours it: tests/test_build_guards.py
                                             disassembles the built library and finds no
                                             v_pk_{add,mul,fma}_f32, and compiles a float2
                                             kernel that has them without the flag
  -ffp-contract=off                          every fma in the kernels is written explicitly, so
                                             the canonical float64 distance is reproduced bit
                                             for bit by the CPU restatement
"""
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT_DIR = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libtrident_hip.so")
SOURCES = ["frontend.hip", "scan.hip", "batch.hip", "cm.hip", "capi.hip"]
# Per-source flags.  batch.hip, cm.hip, frontend.hip: matrix-core results in VGPRs (no
# accumulator-register reads in the per-tile epilogues; the coarse pass gains 13 us at configs[4]);
# batch.hip: no atomic optimizer (it turns the one-lane work-counter atomic into a wave-wide one
# whose result is waited for at once, which would undo taking the next unit early).
EXTRA = {"batch.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1",
                       "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
         "cm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
         "frontend.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
HEADERS = ["common.hpp", "kernels.hpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# what the x86 host pass prints for the device-only feature flag below (see the module doc)
HOST_PASS_NOTE = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-Wall", "-Wno-unused-function",
]


def build(force: bool = True, jobs: int = 3) -> str:
    """Compile every source (in parallel) and link the shared library; returns its path."""
    os.makedirs(OUT_DIR, exist_ok=True)
    deps = [os.path.join(CSRC, h) for h in HEADERS] + [os.path.join(ROOT, "include", "trident_hip.h")]
    newest_dep = max(os.path.getmtime(d) for d in deps)
    procs, objs = [], []
    for s in SOURCES:
        src = os.path.join(CSRC, s)
        obj = os.path.join(OUT_DIR, s.replace(".hip", ".o"))
        objs.append(obj)
        fresh = (os.path.exists(obj) and os.path.getmtime(obj) >= max(os.path.getmtime(src), newest_dep))
        if force or not fresh:
            procs.append((s, subprocess.Popen([HIPCC, *CFLAGS, *EXTRA.get(s, []), "-c", src, "-o", obj],
                                              stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        while len([p for _, p in procs if p.poll() is None]) >= jobs:
            procs[[p.poll() is None for _, p in procs].index(True)][1].wait()
    failed = []
    for name, p in procs:
        log = p.communicate()[0]
        lines = [ln for ln in log.splitlines() if ln.strip() != HOST_PASS_NOTE]
        if lines:
            print("\n".join(lines), file=sys.stderr)
        if p.returncode != 0:
            failed.append(name)
    if failed:
        raise RuntimeError(f"hipcc failed on {', '.join(failed)}")
    tmp = LIB + ".tmp"
    subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(force="--lazy" not in sys.argv))
