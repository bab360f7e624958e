"""Runs the C++ op-surface tests (tests/cpp/test_cuda_ops.cc).

The C++ program exercises include/cuda_ops.h exactly as forward.cc would
call it and checks every result against the CPU oracle; this file only runs
it and reports its output.  Its `cpu` cases need no GPU; its `gpu` cases run
on device 0.
"""
from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "bin", "test_cuda_ops")


def run(group, timeout):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (run __graft_entry__.build())")
    proc = subprocess.run([BIN, group], capture_output=True, text=True, timeout=timeout)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "OK " in proc.stdout


def test_cpp_surface_argument_checks_without_gpu():
    run("cpu", 60)


@pytest.mark.gpu
def test_cpp_surface_on_gpu():
    run("gpu", 120)
