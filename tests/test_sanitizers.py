"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer, on the CPU.

tests/sanitize/Makefile builds, with -fsanitize=address,undefined and no
recovery: the C oracle, the C++ op surface inside its C++ test program, and
(where the reference tree is present) the reference's library minus its
device layer together with this library's host surface in the reference's
test_bench_counters program.  The reference checks its own CPU ops the same
way (CMakeLists.txt:75-85, tests/run_ops_regression.sh of the reference
tree).  Any sanitizer report ends the program with a nonzero status.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.environ.get("MLK_REFERENCE", "/root/reference")
HAVE_REF = os.path.isfile(os.path.join(REF, "src", "forward.cc"))
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=1:halt_on_error=1:abort_on_error=0",
           "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _libasan():
    out = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True)
    path = out.stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


pytestmark = pytest.mark.skipif(_libasan() is None, reason="gcc's AddressSanitizer runtime is absent")


@pytest.fixture(scope="module")
def built(tmp_path_factory):
    out = tmp_path_factory.mktemp("sanitize")
    jobs = str(min(8, os.cpu_count() or 1))
    proc = subprocess.run(["make", "-j" + jobs, "-C", os.path.join(ROOT, "tests", "sanitize"),
                           f"OUT={out}", f"REF={REF}"], capture_output=True, text=True,
                          timeout=900)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-4000:]
    return str(out)


def _clean(text):
    assert "ERROR: AddressSanitizer" not in text and "ERROR: LeakSanitizer" not in text, text[-4000:]
    assert "runtime error:" not in text, text[-4000:]


def test_oracle_tests_under_sanitizers(built):
    """The oracle's CPU tests, with the oracle library swapped for its
    sanitizer build (leak checking off: the Python interpreter itself keeps
    allocations to the end)."""
    lib = os.path.join(built, "liboracle.so")
    env = dict(os.environ, LD_PRELOAD=_libasan(), MLK_ORACLE_LIB=lib,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS=SAN_ENV["UBSAN_OPTIONS"])
    probe = subprocess.run([sys.executable, "-c",
                            "import oracle as O; O.oracle().gather_f32([[1.0]], [0]); "
                            "print(open('/proc/self/maps').read())"],
                           capture_output=True, text=True, env=env, cwd=ROOT, timeout=120)
    assert probe.returncode == 0, probe.stderr[-3000:]
    assert lib in probe.stdout, "the sanitizer build of the oracle was not the one loaded"
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                           os.path.join(ROOT, "tests", "test_oracle.py")],
                          capture_output=True, text=True, env=env, cwd=ROOT, timeout=900)
    _clean(proc.stdout + proc.stderr)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-3000:]


def test_cpp_surface_checks_under_sanitizers(built):
    """The `cpu` group of the C++ op-surface tests (argument checks of every
    entry, host tensors, the KV cache's checks), with leak checking on."""
    proc = subprocess.run([os.path.join(built, "test_cuda_ops"), "cpu"], capture_output=True,
                          text=True, env=dict(os.environ, **SAN_ENV), timeout=300)
    _clean(proc.stdout + proc.stderr)
    assert proc.returncode == 0, proc.stdout[-3000:] + proc.stderr[-3000:]
    assert "OK " in proc.stdout


@pytest.mark.skipif(not HAVE_REF, reason="reference tree not present")
def test_reference_host_code_with_this_library_under_sanitizers(built, tmp_path):
    """The reference's test_bench_counters over its own library (tiny-model
    load, the Q4_0 quantizer over every linear) and this library's host
    surface, all instrumented.  Without a GPU it ends at the first device
    allocation with this library's error; with one it passes."""
    models = tmp_path / "models" / "tiny"
    models.mkdir(parents=True)
    for f in ("model.json", "model.bin"):
        shutil.copy(os.path.join(REF, "model", "tinymodel", f), models / f)
    proc = subprocess.run([os.path.join(built, "test_bench_counters")], capture_output=True,
                          text=True, env=dict(os.environ, **SAN_ENV), cwd=tmp_path, timeout=300)
    out = proc.stdout + proc.stderr
    _clean(out)
    assert "Model loaded successfully" in out
    if proc.returncode != 0:
        assert "cudaSetDevice" in out and "device" in out, out[-3000:]
    else:
        assert "PASS" in proc.stdout
