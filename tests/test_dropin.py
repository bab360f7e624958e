"""The drop-in check on the CPU: the reference's own host library and device
test programs build and link against this library in place of the
reference's device layer, with the reference's headers unchanged.

tests/dropin/Makefile compiles the reference's sources where they lie (every
src/*.cc of its library except the seven src/cuda_*.cc files of its device
layer; CMakeLists.txt:15-48 of the reference tree) into a temporary
directory and links them with -Wl,--no-undefined against
libminilamma_ops.so + libminilamma_hip.so.  It also builds the same sources
with this repository's include/cuda_*.h ahead of the reference's headers,
which fails if a header of this repository shadows one of the reference's
(include/tensor.h, include/model.h, ...), and a layout probe against both
header sets.  Skipped where the reference tree is absent (the GPU box runs
the prebuilt programs, tests/test_gpu_dropin.py).
"""
from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.environ.get("MLK_REFERENCE", "/root/reference")

pytestmark = pytest.mark.skipif(not os.path.isfile(os.path.join(REF, "src", "forward.cc")),
                                reason="reference tree not present")


@pytest.fixture(scope="module")
def built(tmp_path_factory):
    out = tmp_path_factory.mktemp("dropin")
    jobs = str(min(8, os.cpu_count() or 1))
    proc = subprocess.run(["make", "-j" + jobs, "-C", os.path.join(ROOT, "tests", "dropin"),
                           f"OUT={out}", f"REF={REF}"], capture_output=True, text=True,
                          timeout=600)
    assert proc.returncode == 0, proc.stdout[-4000:] + proc.stderr[-4000:]
    return str(out)


def test_no_header_of_this_repository_shadows_the_reference():
    ours = set(os.listdir(os.path.join(ROOT, "include")))
    theirs = set(os.listdir(os.path.join(REF, "include")))
    # only the device layer's headers may share a name with the reference's
    shared = {h for h in ours & theirs if not h.startswith("cuda_")}
    assert not shared, sorted(shared)


def test_reference_library_links_with_no_undefined_symbols(built):
    # -Wl,--no-undefined: the library's exports cover everything the
    # reference's code calls in its device layer, including the thread-local
    # internal::active_cuda_stats of src/internal/cuda_stats.h
    for name in ("libyan_minillama.so", "libyan_minillama_overlay.so"):
        assert os.path.isfile(os.path.join(built, "lib", name)), name
    undefined = subprocess.run(["nm", "-DC", "--undefined-only",
                                os.path.join(built, "lib", "libyan_minillama.so")],
                               capture_output=True, text=True, check=True).stdout
    assert "yan_lamma::internal::active_cuda_stats" in undefined
    exported = subprocess.run(["nm", "-DC", "--defined-only", os.path.join(
        ROOT, "cpp-minilamma_amd", "lib", "libminilamma_ops.so")],
        capture_output=True, text=True, check=True).stdout
    assert "yan_lamma::internal::active_cuda_stats" in exported


def test_layouts_agree_with_the_reference_headers(built):
    ref = subprocess.run([os.path.join(built, "bin", "layout_ref")], capture_output=True,
                         text=True, check=True).stdout
    lib = subprocess.run([os.path.join(built, "bin", "layout_lib")], capture_output=True,
                         text=True, check=True).stdout
    assert ref.splitlines() == lib.splitlines()
    assert "CudaModelWeights.host_to_device_copies" in ref


def test_reference_test_programs_reach_this_library(built):
    # without a GPU the programs get as far as this library's device count:
    # CudaRuntimeBuilt() is true and DeviceCount() reports no device.
    # test_forward_batch is the reference-side binding of the batched layer
    # (tests/dropin/forward_batch_device.cc) with its test, built against the
    # reference's headers and linked with its library
    for prog in ("test_cuda_runtime", "test_cuda_ops", "test_cuda_forward",
                 "test_forward_batch"):
        proc = subprocess.run([os.path.join(built, "bin", prog)],
                              capture_output=True, text=True, timeout=60, cwd=built)
        if proc.returncode == 0:  # a machine with a GPU: the program passed
            assert "PASS" in proc.stdout
        else:
            assert "requires an available device" in proc.stderr, proc.stderr
