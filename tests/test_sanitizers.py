"""AddressSanitizer + UndefinedBehaviorSanitizer runs of the CPU code: the
C++ host mirror's CPU checks (tests/cpp/host_test cpu) and the oracle's own
test file, against g++/gcc sanitizer builds made by tests/cpp/build.py
(build_sanitized). Device code is never built with a sanitizer; the HIP
library is loaded unsanitized and, without a GPU, only its argument checks
and no-device paths run. Leak detection is off: the HIP runtime keeps
process-lifetime allocations."""
import importlib.util
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def _libasan():
    p = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True,
                       check=True).stdout.strip()
    if not os.path.isabs(p):
        pytest.skip("gcc has no libasan")
    return p


@pytest.fixture(scope="module")
def san(tmp_path_factory):
    spec = importlib.util.spec_from_file_location("hbuild", os.path.join(HERE, "cpp", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.build_sanitized(str(tmp_path_factory.mktemp("san")))


def _env(extra=None):
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=0:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env.update(extra or {})
    return env


def test_host_mirror_cpu_under_sanitizers(san):
    r = subprocess.run([san["host_test"], "cpu"], capture_output=True, text=True, timeout=600,
                       env=_env())
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr


def test_oracle_under_sanitizers(san):
    env = _env({"LD_PRELOAD": _libasan(), "GONN_ORACLE_LIB": san["oracle"],
                "PYTHONPATH": ROOT, "OMP_NUM_THREADS": "4"})
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        os.path.join(HERE, "test_oracle.py"), "-k", "not planted"],
                       capture_output=True, text=True, timeout=900, env=env, cwd=ROOT)
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-4000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr
