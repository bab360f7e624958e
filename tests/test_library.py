"""CPU checks of the product libraries: they load, export every symbol the
headers declare, and reject bad arguments before touching a device (no
kernel is launched here)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import __graft_entry__ as entry
from conftest import load_workloads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(ROOT, "cpp-minilamma_amd", "lib")


def declared_c_functions():
    text = open(os.path.join(INCLUDE, "minilamma_hip.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int64_t|int|mlk_status)\s+(mlk_\w+)\(",
                                 text, flags=re.M)))


def dynamic_symbols(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_hip_library_exports_every_declared_function():
    names = declared_c_functions()
    assert len(names) >= 30
    syms = dynamic_symbols(os.path.join(LIB, "libminilamma_hip.so"))
    missing = [n for n in names if n not in syms]
    assert not missing, missing
    mlk = entry.load_package()
    assert sorted(mlk.exported_symbols()) == names, "binding and header disagree"
    for n in names:
        getattr(mlk.lib, n)


def test_hip_library_is_built_for_gfx950_only():
    strings = subprocess.run(["strings", os.path.join(LIB, "libminilamma_hip.so")],
                             capture_output=True, text=True, check=True).stdout
    targets = set(re.findall(r"amdgcn-amd-amdhsa--(gfx\w+)", strings))
    assert targets == {"gfx950"}, targets


CPP_SURFACE = [
    "CudaopsBuild", "CudaEmbeddingDevice", "CudaRmsNormHost", "CudaRmsNromDevice", "CudaSilu",
    "CudaSiluDevice", "CudaElementwiseMul", "CudaElementwiseMulDevice", "CudaElementAddDevice",
    "OCudaElementAddDevice", "CudaSoftmax", "CudaRopeHost", "CudaRopeDevice",
    "CudaAddRmsNormDevice", "CudaRmsNormRowsDevice", "CudaSwiGluDevice", "CudaRopeBatchDevice",
    "CudaRopeRangeDevice", "CudaEmbeddingBatchDevice", "CudaEmbeddingQuantDevice",
    "CudaQuantizeDevice", "CudaRuntimeBuilt", "GetCudaInfo", "DeviceCount", "SetCudaService",
    "CudaMemory", "CudaFreeMemory", "CudaMemcpy", "CudaEmptyCache", "CudaCachedBytes",
    "TensorHostToDevice",
    # include/cuda_matmul.h, include/cuda_quant.h
    "cuBLASBuilt", "CudaMatmul", "CudaLinear", "CudaLinearHostDevice", "CudaLinearDevice",
    "CudaQuantBuilt", "CudaQ40Linear", "CudaQ40DeviceLinear", "CudaQ40DeviceInputLinear",
    "CudaQ41Linear", "CudaQ41DeviceLinear", "CudaQ41DeviceInputLinear", "CudaQ80Linear",
    "CudaQ80DeviceLinear", "CudaQ80DeviceInputLinear",
    # include/cuda_kvcache.h, include/cuda_attention.h
    "CudaCacheBuild", "CudaCache::Reset", "CudaCache::WriteHost", "CudaCache::WriteDevice",
    "CudaCache::ReadKey", "CudaCache::ReadVal", "CudaCache::ReadHeadKey", "CudaCache::ReadHeadVal",
    "CudaCache::KData", "CudaCache::vData", "CudaCache::Bytes_", "CudaCache::Clear",
    "CudaCache::SlotOffsetBytes", "CudaKvWriteBatchDevice", "CudaAttentionBuilt",
    "CudaAttentionDecode", "CudaAttentionDevice", "CudaAttentionBatchDevice",
    # include/cuda_forward.h
    "CudaForwardLayerBatchDevice",
]


def test_op_surface_library_exports_the_reference_ops():
    out = subprocess.run(["nm", "-DC", "--defined-only", os.path.join(LIB, "libminilamma_ops.so")],
                         capture_output=True, text=True, check=True).stdout
    for name in CPP_SURFACE:
        assert re.search(r"yan_lamma::" + name + r"\(", out), name
    # the op surface carries no HIP headers: nothing from the HIP runtime is
    # referenced directly, only the C ABI
    undef = subprocess.run(["nm", "-D", "--undefined-only",
                            os.path.join(LIB, "libminilamma_ops.so")],
                           capture_output=True, text=True, check=True).stdout
    assert "hipMalloc" not in undef and "mlk_malloc" in undef


def test_host_sources_include_no_hip_header():
    host = os.path.join(ROOT, "cpp-minilamma_amd", "host")
    for top, _, files in os.walk(host):
        for f in files:
            text = open(os.path.join(top, f)).read()
            assert "hip_runtime" not in text and "cuda_runtime_api" not in text, f


def test_validation_happens_before_any_device_call():
    mlk = entry.load_package()
    fake = 4096  # never dereferenced: every call below must fail validation first
    cases = [
        (lambda: mlk.add_rmsnorm(fake, None, fake, fake, 1, 4, 0.0), "eps must be finite"),
        (lambda: mlk.add_rmsnorm(fake, None, None, fake, 1, 4, 1e-5), "must not be null"),
        (lambda: mlk.add_rmsnorm(fake, None, fake, fake, 0, 4, 1e-5), "must be positive"),
        (lambda: mlk.add_rmsnorm(fake, fake + 64, fake, fake, 1, 4, 1e-5), "alias"),
        (lambda: mlk.swiglu(fake, fake, fake, 0), "must not be empty"),
        (lambda: mlk.swiglu(None, fake, fake, 4), "must not be null"),
        (lambda: mlk.rope(fake, fake, 1, 2, 1, 3, pos0=0), "head_dim must be positive and even"),
        (lambda: mlk.rope(fake, fake, 1, 2, 1, 4, pos0=-1), "pos must be non-negative"),
        (lambda: mlk.rope(fake, fake, 1, 2, 1, 4, pos0=0, theta=0.0), "theta must be finite"),
        (lambda: mlk.rope(fake, fake, 1, 2, 1, 4, pos0=0, q_row_stride=4), "row strides"),
        (lambda: mlk.rope(fake, fake, 1, 2, 1, 4, pos0=0, rope_type=7), "unknown rope type"),
        (lambda: mlk.rope(fake, fake, 2, 2, 1, 4, pos0=2 ** 31 - 1), "int32 range"),
        (lambda: mlk.gather_f32(fake, 4, 4, None, 1, fake, token=4), "token_id must be in"),
        (lambda: mlk.gather_f32(fake, 4, 4, None, 2, fake, token=0), "exactly one row"),
        (lambda: mlk.gather_f32(fake, 0, 4, None, 1, fake, token=0), "must be positive"),
        (lambda: mlk.gather_quant("q8_0", None, 4, 4, None, 1, fake), "must not be null"),
        (lambda: mlk.quantize("q4_1", fake, 0, 32, fake), "must be positive"),
        (lambda: mlk.quantize("q4_1", fake, 1, 32, fake + 1), "2-byte aligned"),
        (lambda: mlk.softmax(fake, fake, 1, 4), "alias"),
        (lambda: mlk.softmax(fake, fake + 64, 0, 4), "must not be empty"),
        (lambda: mlk.linear_quant("q8_0", fake, fake + 64, fake + 128, 0, 32, 4),
         "must be positive"),
        (lambda: mlk.linear_quant("q8_0", None, fake, fake + 64, 1, 32, 4), "must not be null"),
        (lambda: mlk.linear_quant("q4_0", fake, fake + 64, fake, 1, 32, 4), "alias"),
        (lambda: mlk.linear_quant("q4_1", fake, fake + 1, fake + 64, 1, 32, 4), "2-byte aligned"),
        (lambda: mlk.linear_f32(fake, fake + 64, fake + 128, 1, 0, 4), "must be positive"),
        (lambda: mlk.linear_f32(fake, fake + 64, fake + 2, 1, 4, 4), "4-byte aligned"),
        (lambda: mlk.matmul(fake, fake + 64, fake, 2, 2, 2), "alias"),
        (lambda: mlk.matmul(fake, fake + 64, fake + 128, 2, 0, 2), "must be positive"),
    ]
    for call, text in cases:
        with pytest.raises(mlk.MlkError, match=text):
            call()
    # unknown quantization type goes straight through the C ABI
    assert mlk.lib.mlk_gather_quant(9, None, 1, 1, None, 0, 1, None, None, None) == \
        mlk.MLK_ERR_INVALID
    assert b"unknown quantization type" in mlk.lib.mlk_last_error()
    assert mlk.lib.mlk_linear_quant(3, None, None, None, None, 1, 1, 1, None, 0, None) == \
        mlk.MLK_ERR_INVALID


def test_quant_bytes_and_status_strings():
    mlk = entry.load_package()
    assert mlk.quant_bytes("q8_0", 128256, 4096) == 128256 * 128 * 34
    assert mlk.quant_bytes("q4_0", 2, 33) == 2 * 2 * 18
    assert mlk.quant_bytes("q4_1", 1, 32) == 20
    assert mlk.lib.mlk_quant_bytes(5, 1, 32) == 0
    assert mlk.lib.mlk_status_string(0) == b"success"
    assert mlk.lib.mlk_abi_version() == 2


def test_no_gpu_here_reports_zero_devices_or_a_hip_error():
    mlk = entry.load_package()
    n = ctypes.c_int(-1)
    st = mlk.lib.mlk_device_count(ctypes.byref(n))
    assert st in (mlk.MLK_OK, mlk.MLK_ERR_HIP)
    if st == mlk.MLK_OK:
        assert n.value >= 0


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr


def test_workload_byte_counts_match_the_baseline_table():
    w = load_workloads()
    c3 = w.CONFIGS["c3_prefill_8b"]
    c5 = w.CONFIGS["c5_70b"]
    assert w.bytes_add_rmsnorm(4096, 4096) == 268_451_840
    assert w.bytes_add_rmsnorm(8192, 8192) == 1_073_774_592
    assert w.bytes_swiglu(4096, 14336) == 704_643_072
    assert w.bytes_swiglu(8192, 28672) == 2_818_572_288
    assert w.bytes_rope(4096, 32, 8, 128) == 167_772_160
    assert w.bytes_rope(8192, 64, 8, 128) == 603_979_776
    assert w.bytes_gather_f32(4096, 4096) == 134_234_112
    assert w.bytes_gather_quant("q8_0", 4096, 4096) == 84_951_040
    assert w.bytes_gather_quant("q4_0", 4096, 4096) == 76_562_432
    assert w.bytes_gather_quant("q4_1", 4096, 4096) == 77_611_008
    assert w.bytes_chain(c3, 4096) == 1_275_101_184
    assert w.bytes_chain(c5, 8192, with_gather=False) == 4_496_326_656


def test_zipf_ids_are_deterministic_and_in_range():
    w = load_workloads()
    a = w.zipf_ids(4096, 128256, 1.1, 7)
    b = w.zipf_ids(4096, 128256, 1.1, 7)
    assert a.dtype == np.int32 and (a == b).all()
    assert a.min() >= 0 and a.max() < 128256
    # Zipf: id 0 is the most frequent and the ranks decay
    counts = np.bincount(a, minlength=10)
    assert counts[0] == counts.max() and counts[0] > counts[9]


def test_unique_row_bytes_count_each_distinct_row_once():
    w = load_workloads()
    ids = np.array([5, 5, 5, 9, 0], np.int32)
    # 3 distinct rows read, 5 rows written, 5 ids
    assert w.bytes_gather_unique(ids, 64) == 3 * 256 + 5 * 256 + 20
    assert w.bytes_gather_unique(ids, 64, "q8_0") == 3 * 2 * 34 + 5 * 256 + 20
    # with no repeats it is the algorithmic figure
    ids = np.arange(7, dtype=np.int32)
    assert w.bytes_gather_unique(ids, 4096) == w.bytes_gather_f32(7, 4096)
    assert w.bytes_gather_unique(ids, 4096, "q4_1") == w.bytes_gather_quant("q4_1", 7, 4096)
