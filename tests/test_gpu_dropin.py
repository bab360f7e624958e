"""The reference's own device test suite, run on the GPU against this library.

The programs are the reference's tests/test_cuda_<part>.cc and
test_bench_counters.cc, compiled from the reference's sources and linked
against libminilamma_ops.so + libminilamma_hip.so in place of the
reference's device layer (tests/dropin/Makefile, built in the container that
holds the reference tree; the GPU box runs the prebuilt programs).  The
cases and their modes are the reference's CTest list
(tests/CMakeLists.txt:14-29, 46), run from a directory that holds the tiny
model where its tests look for it (models/tiny, tests/cuda_test_support.h:49).  Each
program prints "PASS <mode> CUDA" per case and exits 0 only if every check
passed; the forward cases compare the device logits with the CPU forward
pass token by token and check the transfer counters: no host-to-device
copy and one 524-byte logits download per token
(tests/cuda_test_support.h:88-125).
"""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "tests", "dropin", "_build")

# (CTest name, program, mode) from tests/CMakeLists.txt:14-31 and :47-50
CASES = [
    ("cuda_runtime", "test_cuda_runtime", "runtime"),
    ("cuda_matmul", "test_cuda_matmul", "matmul"),
    ("cuda_linear", "test_cuda_linear", "f32"),
    ("cuda_quant_q8_0", "test_cuda_quant", "q8_0"),
    ("cuda_quant_q4", "test_cuda_quant", "q4"),
    ("cuda_ops", "test_cuda_ops", "ops"),
    ("cuda_kv_cache", "test_cuda_kv_cache", "kv"),
    ("cuda_attention", "test_cuda_attention", "direct"),
    ("cuda_kv_attention", "test_cuda_attention", "kv"),
    ("cuda_forward_attention", "test_cuda_attention", "forward"),
    ("cuda_forward", "test_cuda_forward", "forward"),
    ("cuda_forward_quant", "test_cuda_quant", "forward"),
    ("cuda_forward_q4", "test_cuda_quant", "forward_q4"),
    ("cuda_forward_buffer", "test_cuda_forward_buffer", "f32"),
    ("cuda_forward_device_resident", "test_cuda_forward_buffer", "q8_0"),
    ("cuda_forward_linear", "test_cuda_forward_linear", "linear"),
    ("strict-bench-counters", "test_bench_counters", None),
]

# The reference-side binding of the batched layer and of the device token
# table (tests/dropin/forward_batch_device.cc), held to the reference's
# device-forward bar against its CPU ForwardBatch with the transfer counters
# (tests/dropin/test_forward_batch.cc): linears F32 / Q8_0 / Q4_0 with the F32
# table, the token table as Q8_0 / Q4_0 / Q4_1 blocks, the token-loop
# fallback for positions that do not increase, and the rejected calls.
BINDING_MODES = ["f32", "q8_0", "q4_0", "table_q8_0", "table_q4_0", "table_q4_1", "fallback",
                 "rejects"]
CASES += [(f"forward_batch_device_{m}", "test_forward_batch", m) for m in BINDING_MODES]


@pytest.mark.gpu
@pytest.mark.parametrize("name,program,mode", CASES, ids=[c[0] for c in CASES])
def test_reference_device_suite(name, program, mode):
    exe = os.path.join(BUILD, "bin", program)
    if not os.path.isfile(exe):
        pytest.skip("drop-in programs not built (tests/dropin/Makefile needs the reference tree)")
    cmd = [exe] + ([mode] if mode else [])
    print(f"drop-in case {name}: {' '.join(cmd)}", flush=True)
    sys.stdout.flush()
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=120, cwd=BUILD)
    print(proc.stdout[-3000:])
    assert proc.returncode == 0, f"{name}: rc={proc.returncode}\n{proc.stdout[-3000:]}\n{proc.stderr[-3000:]}"
    if mode:
        assert f"PASS {mode} CUDA" in proc.stdout, proc.stdout
