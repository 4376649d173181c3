"""Build recipe for the oracle (test infrastructure, not product code).

Compiles oracle/attn_oracle.c into oracle/liboracle.so with gcc. The flags keep
IEEE fp64 semantics (no -ffast-math, no FMA contraction) so results do not
depend on the host CPU; OpenMP only splits independent rows.

The reference's own attention path cannot be compiled here: it is Go
(nn/attention.go + tensor/ + gonum, no Go toolchain in the image) and CUDA
(backend/cuda/gonn_cuda.cu, no nvcc), so there is no oracle/_ref build.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "attn_oracle.c")
OUT = os.path.join(HERE, "liboracle.so")


def build(verbose: bool = False) -> str:
    cmd = ["gcc", "-O3", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math",
           "-fopenmp", "-fPIC", "-shared", "-o", OUT + ".tmp", SRC, "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
