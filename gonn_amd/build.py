"""Build libgonn_hip.so for gfx950 in-tree (gonn_amd/libgonn_hip.so).

    python -m gonn_amd.build          # or: python gonn_amd/build.py

Every .hip file under gonn_amd/csrc is compiled with hipcc for gfx950 only and
linked into one shared library exposing the C ABI of include/gonn_hip.h. The
C++ host mirror of GoNN's attention seam (gonn_amd/host/*.cpp) is built on
top of it as gonn_amd/libgonn_host.so.
Packed-fp32 VALU instructions are disabled for device code; hipcc's host pass
reports that feature as unknown, which is harmless.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libgonn_hip.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", CSRC, "-I", os.path.join(os.path.dirname(HERE), "include"),
]


# Per-file device flags. The forward kernels take row maxima of MFMA results
# with fmaxf; in the default IEEE mode every operand is first canonicalised
# (one extra v_max per operand) and v_max3 is not formed. No value on that
# path is NaN (masked scores are -inf), so the file is built with relaxed NaN
# handling and the IEEE mode bit off, which turns the reductions into v_max3.
FILE_FLAGS = {
    "attn_fwd.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"],
    # MFMAs with VGPR accumulators (the score tiles the VALU reads); the file
    # header gives the reason.
    "attn_bwd_dq.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *CFLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed for {src}")
    warn = "\n".join(x for x in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in x and x.strip())
    if warn and verbose:
        print(warn)
    return obj


HOST_LIB = os.path.join(HERE, "libgonn_host.so")
HOST_SRC = os.path.join(HERE, "host")


def build_host(verbose: bool = False) -> str:
    """The C++ host mirror of GoNN's attention seam (gonn_amd/host) as
    libgonn_host.so, linked against libgonn_hip.so (found next to it)."""
    srcs = sorted(os.path.join(HOST_SRC, f) for f in os.listdir(HOST_SRC) if f.endswith(".cpp"))
    tmp = HOST_LIB + ".tmp"
    cmd = ["g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", "-pthread",
           "-I", HOST_SRC, "-I", os.path.join(os.path.dirname(HERE), "include"), *srcs,
           "-L", HERE, "-lgonn_hip", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
           "-L/opt/rocm/lib", "-lrocblas", "-Wl,-rpath,/opt/rocm/lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    build_host(verbose)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
