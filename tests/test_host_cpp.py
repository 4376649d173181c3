"""The C++ host mirror of GoNN's attention seam (gonn_amd/host, built as
gonn_amd/libgonn_host.so), driven by tests/cpp/host_test.

CPU: argument checks, shape ops, Linear vs the oracle, the no-device error
path. GPU: MultiHeadAttention Forward / ForwardFused (config C1 and
variants) vs the oracle's MHA and fusedAttnDiff gradients vs the oracle's
autograd, in both MFMA modes (tolerances in tests/cpp/host_test.cpp)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "host_test")


def _run(mode):
    if not os.path.exists(BIN):
        if mode == "gpu":
            pytest.fail("tests/cpp/host_test is not built; run __graft_entry__.build()")
        import importlib.util
        spec = importlib.util.spec_from_file_location("hbuild", os.path.join(HERE, "cpp", "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    r = subprocess.run([BIN, mode], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_host_cpp_cpu():
    _run("cpu")


@pytest.mark.gpu
def test_host_cpp_gpu():
    _run("gpu")
