"""Build recipe for the CPU oracle (test infrastructure only).

Compiles oracle/trident_oracle.c into oracle/liboracle.so with gcc + OpenMP.
``-ffp-contract=off`` keeps every floating-point operation exactly as written, so the
canonical float64 distance (explicit ``fma`` in dimension order) is reproduced bit for
bit.  ``-march=x86-64-v3`` (AVX2 + FMA) keeps the binary portable to the GPU hosts.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "trident_oracle.c")
LIB = os.path.join(HERE, "liboracle.so")


def build(force: bool = True) -> str:
    if not force and os.path.exists(LIB) and os.path.getmtime(LIB) >= os.path.getmtime(SRC):
        return LIB
    tmp = LIB + ".tmp"
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fopenmp", "-fPIC",
           "-shared", "-o", tmp, SRC, "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(force="--lazy" not in sys.argv))
