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


SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
       "-fno-omit-frame-pointer", "-g", "-O1"]


def build_sanitized(outdir: str, verbose: bool = False) -> dict:
    """AddressSanitizer + UndefinedBehaviorSanitizer builds of the CPU code
    into outdir, all with g++/gcc on the host (no device code is built with a
    sanitizer): the oracle (liboracle.so), the C++ host mirror
    (libgonn_host.so, linked against the in-tree libgonn_hip.so) and this
    driver (host_test). Returns their paths."""
    pkg, orc = os.path.join(ROOT, "gonn_amd"), os.path.join(ROOT, "oracle")
    os.makedirs(outdir, exist_ok=True)
    lib_o = os.path.join(outdir, "liboracle.so")
    lib_h = os.path.join(outdir, "libgonn_host.so")
    exe = os.path.join(outdir, "host_test")
    hsrc = sorted(os.path.join(pkg, "host", f) for f in os.listdir(os.path.join(pkg, "host"))
                  if f.endswith(".cpp"))
    cmds = [
        ["gcc", *SAN, "-ffp-contract=off", "-fopenmp", "-fPIC", "-shared", "-o", lib_o,
         os.path.join(orc, "attn_oracle.c"), "-lm"],
        ["g++", "-std=c++17", *SAN, "-fPIC", "-shared", "-pthread", "-I", os.path.join(pkg, "host"),
         "-I", os.path.join(ROOT, "include"), *hsrc, "-o", lib_h, "-L", pkg, "-lgonn_hip",
         f"-Wl,-rpath,{pkg}"],
        ["g++", "-std=c++17", *SAN, "-pthread", "-I", os.path.join(pkg, "host"),
         "-I", os.path.join(ROOT, "include"), os.path.join(HERE, "host_test.cpp"), "-o", exe,
         "-L", outdir, "-lgonn_host", "-loracle", "-L", pkg, "-lgonn_hip",
         f"-Wl,-rpath,{outdir}", f"-Wl,-rpath,{pkg}"],
    ]
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd))
        subprocess.run(cmd, check=True)
    return {"oracle": lib_o, "host": lib_h, "host_test": exe}


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
