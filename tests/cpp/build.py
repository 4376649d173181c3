"""Build tests/cpp/host_test, the test driver of the C++ host mirror
(gonn_amd/libgonn_host.so). It links the fp64 oracle (oracle/liboracle.so)
as its checker. Test infrastructure: run by __graft_entry__.build() after the
library and the oracle are built."""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
OUT = os.path.join(HERE, "host_test")


def build(verbose: bool = False) -> str:
    pkg, orc = os.path.join(ROOT, "gonn_amd"), os.path.join(ROOT, "oracle")
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-pthread",
           "-I", os.path.join(pkg, "host"), "-I", os.path.join(ROOT, "include"),
           os.path.join(HERE, "host_test.cpp"), "-o", OUT + ".tmp",
           "-L", pkg, "-lgonn_host", "-lgonn_hip", "-L", orc, "-loracle",
           f"-Wl,-rpath,{pkg}", f"-Wl,-rpath,{orc}",
           "-Wl,-rpath,$ORIGIN/../../gonn_amd", "-Wl,-rpath,$ORIGIN/../../oracle"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(OUT + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
