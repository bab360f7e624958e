"""Shared pytest setup.

Markers: `gpu` tests need an MI355X and the built HIP library; everything
else runs on the CPU (oracle vs golden fixtures and the compiled reference,
host logic, library loading and exported symbols).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def load_workloads():
    """cpp-minilamma_amd/workloads.py (pure Python: importable without the
    built HIP library)."""
    import importlib.util
    name = "cpp_minilamma_amd_workloads"
    if name not in sys.modules:
        spec = importlib.util.spec_from_file_location(
            name, os.path.join(ROOT, "cpp-minilamma_amd", "workloads.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        sys.modules[name] = mod
    return sys.modules[name]


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def orc():
    import oracle as O
    return O.oracle()


@pytest.fixture(scope="session")
def mlk():
    """The HIP package, with device 0 selected; fails loudly if it is missing."""
    import __graft_entry__ as g
    pkg = g.load_package()
    pkg.set_device(0)
    return pkg


def golden(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def tiny_model():
    """The reference's tiny model and its own forward-pass logits
    (tests/golden/tiny_forward.npz) as (model, tokens, positions, logits) in
    oracle.forward_model layout."""
    g = golden("tiny_forward")
    keys = ("vocab", "dim", "hidden_dim", "layers", "n_heads", "n_kv_heads", "head_dim",
            "max_seq", "rope_type")
    config = {k: int(v) for k, v in zip(keys, g["config"])}
    config["theta"], config["eps"] = (float(v) for v in g["theta_eps"])
    layers = []
    for i in range(config["layers"]):
        lw = {n: g[f"l{i}_{n}"] for n in ("attention_norm", "ffn_norm")}
        for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            lw[n] = ("f32", g[f"l{i}_{n}"])
        layers.append(lw)
    model = {"config": config, "embedding": g["embedding"], "layers": layers,
             "final_norm": g["final_norm"], "lm_head": ("f32", g["lm_head"])}
    return model, g["tokens"], g["positions"], g["logits"]


def assert_bits_equal(got, want, what="", nan_equal=False):
    got = np.ascontiguousarray(got, dtype=np.float32)
    want = np.ascontiguousarray(want, dtype=np.float32)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    diff = got.view(np.uint32) != want.view(np.uint32)
    if nan_equal:
        diff &= ~(np.isnan(got) & np.isnan(want))
    if diff.any():
        i = int(np.flatnonzero(diff.reshape(-1))[0])
        raise AssertionError(f"{what}: {int(diff.sum())} elements differ, first at {i}: "
                             f"{got.reshape(-1)[i]!r} vs {want.reshape(-1)[i]!r}")


def assert_terms_close(got, want, terms_abs, what="", rtol=1e-5):
    """The reference's bar: |got - want| <= 1e-5 * max(1, sum|terms|)
    (README.md:7, test/ops_test.cc:520-521).  terms_abs is sum|terms| per
    element (same shape as want)."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    bound = rtol * np.maximum(1.0, np.asarray(terms_abs, dtype=np.float64))
    err = np.abs(got - want)
    bad = err > bound
    if bad.any():
        i = int(np.flatnonzero(bad.reshape(-1))[0])
        raise AssertionError(f"{what}: {int(bad.sum())} elements beyond tolerance, first at {i}: "
                             f"{got.reshape(-1)[i]!r} vs {want.reshape(-1)[i]!r}")


def max_ulp(got, want):
    a = np.ascontiguousarray(got, dtype=np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(want, dtype=np.float32).view(np.int32).astype(np.int64)
    return int(np.abs(a - b).max()) if a.size else 0


U32 = 2.0 ** -24  # float32 unit roundoff


def dot_exact(x, w, bias=None):
    """float64 value and sum of |terms| of x @ w^T (+ bias) for x [T, K],
    w [O, K]."""
    x64 = np.atleast_2d(np.asarray(x, np.float64))
    w64 = np.asarray(w, np.float64)
    y = x64 @ w64.T
    s = np.abs(x64) @ np.abs(w64).T
    if bias is not None:
        b = np.asarray(bias, np.float64)
        y, s = y + b, s + np.abs(b)
    return y, s


def assert_dot_close(got, exact, abs_terms, n_terms, what=""):
    """The linear-layer bar: any fp32 summation order of n terms is within
    gamma_n * sum|terms| of the exact value (Higham, Accuracy and Stability
    of Numerical Algorithms, eq. 3.8); the reference's serial loop and the
    kernels are held to the same bound."""
    got = np.atleast_2d(np.asarray(got, np.float64))
    gamma = n_terms * U32 / (1 - n_terms * U32)
    err = np.abs(got - exact)
    lim = gamma * abs_terms
    bad = ~(err <= lim)
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {got.size} outside gamma_{n_terms} bound; "
                           f"worst err {float(err.max()):.3e} vs bound {float(lim.min()):.3e}")
