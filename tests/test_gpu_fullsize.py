"""GPU parity at BASELINE.json's full configuration sizes.

Inputs are generated on the device (the same generator bench.py uses),
downloaded, and the oracle recomputes every output element on the CPU: the
C oracle finishes even the 70B SwiGLU (235M elements) in a few seconds.
Bars as in test_gpu_ops.py: gathers, quantizer and residual add bit-exact;
RMSNorm / RoPE / SwiGLU within 1e-5 * max(1, sum|terms|).  Size-independent
properties are checked beside: RoPE preserves every head's norm, the
quantized gather equals the dequantized table rows.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import (assert_bits_equal, assert_dot_close, assert_terms_close, dot_exact,
                      load_workloads, max_ulp)

W = load_workloads()

pytestmark = pytest.mark.gpu


def ulp_report(what, got, want):
    """Prints the distribution of ulp distances to the oracle (run pytest -s)."""
    a = np.ascontiguousarray(got, np.float32).view(np.int32).astype(np.int64).reshape(-1)
    b = np.ascontiguousarray(want, np.float32).view(np.int32).astype(np.int64).reshape(-1)
    d = np.abs(a - b)
    print(f"ULP {what}: n={d.size} exact={np.mean(d == 0):.6f} <=1ulp={np.mean(d <= 1):.6f} "
          f"max={int(d.max())} max_abs_err={float(np.abs(got - want).max()):.3e}")


def device_normal(mlk, shape, mean, std, seed):
    buf = mlk.DeviceBuffer.empty(shape)
    mlk.fill_normal(buf, int(np.prod(shape)), mean, std, seed)
    return buf


@pytest.mark.parametrize("name", ["c3_prefill_8b", "c5_70b"])
def test_add_rmsnorm_full_size(mlk, orc, name):
    cfg = W.CONFIGS[name]
    T, D = cfg["tokens"], cfg["dim"]
    x = device_normal(mlk, (T, D), 0.0, 0.02, cfg["seed"] + 1)
    d = device_normal(mlk, (T, D), 0.0, 0.02, cfg["seed"] + 2)
    w = device_normal(mlk, (D,), 1.0, 0.1, cfg["seed"] + 3)
    hx, hd, hw = x.download(), d.download(), w.download()
    y = mlk.DeviceBuffer.empty((T, D))
    mlk.add_rmsnorm(x, d, w, y, T, D, cfg["eps"])
    er, ey = orc.add_rmsnorm(hx, hd, hw, cfg["eps"])
    assert_bits_equal(x.download(), er, f"{name} residual")
    got = y.download()
    assert_terms_close(got, ey, np.abs(ey), f"{name} rmsnorm")
    ulp_report(f"{name} rmsnorm", got, ey)


@pytest.mark.parametrize("name", ["c3_prefill_8b", "c5_70b"])
def test_swiglu_full_size(mlk, orc, name):
    cfg = W.CONFIGS[name]
    T, F = cfg["tokens"], cfg["ffn"]
    g = device_normal(mlk, (T, F), 0.0, 0.02, cfg["seed"] + 4)
    u = device_normal(mlk, (T, F), 0.0, 0.02, cfg["seed"] + 5)
    y = mlk.DeviceBuffer.empty((T, F))
    mlk.swiglu(g, u, y, T * F)
    hg, hu = g.download(), u.download()
    del g, u
    exp = orc.swiglu(hg, hu)
    got = y.download()
    assert_terms_close(got, exp, np.abs(exp), f"{name} swiglu")
    ulp_report(f"{name} swiglu", got, exp)


@pytest.mark.parametrize("name", ["c3_prefill_8b", "c5_70b"])
def test_rope_full_size(mlk, orc, name):
    cfg = W.CONFIGS[name]
    T, H, KV, hd = cfg["tokens"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    q = device_normal(mlk, (T, H * hd), 0.0, 0.02, cfg["seed"] + 6)
    k = device_normal(mlk, (T, KV * hd), 0.0, 0.02, cfg["seed"] + 7)
    hq, hk = q.download(), k.download()
    mlk.rope(q, k, T, H, KV, hd, pos0=0, theta=cfg["theta"])
    gq, gk = q.download(), k.download()
    eq, ek = orc.rope(hq, hk, H, KV, hd, pos0=0, theta=cfg["theta"])
    assert_terms_close(gq, eq, np.abs(eq), f"{name} rope q")
    assert_terms_close(gk, ek, np.abs(ek), f"{name} rope k")
    ulp_report(f"{name} rope q", gq, eq)
    ulp_report(f"{name} rope k", gk, ek)
    # a rotation keeps every head's norm
    for before, after, heads in ((hq, gq, H), (hk, gk, KV)):
        n0 = (before.reshape(T, heads, hd).astype(np.float64) ** 2).sum(-1)
        n1 = (after.reshape(T, heads, hd).astype(np.float64) ** 2).sum(-1)
        np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-12)


def test_gather_f32_full_size(mlk, orc):
    cfg = W.CONFIGS["c3_prefill_8b"]
    T, V, D = cfg["tokens"], cfg["vocab"], cfg["dim"]
    table = device_normal(mlk, (V, D), 0.0, 0.02, cfg["seed"])
    ids = W.zipf_ids(T, V, 1.1, cfg["seed"])
    ids[:2] = [0, V - 1]
    d_ids = mlk.DeviceBuffer.from_array(ids)
    out = mlk.DeviceBuffer.empty((T, D))
    mlk.gather_f32(table, V, D, d_ids, T, out)
    assert_bits_equal(out.download(), orc.gather_f32(table.download(), ids), "gather")


@pytest.mark.parametrize("qtype", ["q8_0", "q4_0", "q4_1"])
def test_quantized_gather_full_size(mlk, orc, qtype):
    cfg = W.CONFIGS["c4_quant_gather"]
    T, V, D = cfg["tokens"], cfg["vocab"], cfg["dim"]
    table = device_normal(mlk, (V, D), 0.0, 0.02, cfg["seed"])
    blocks = mlk.DeviceBuffer(mlk.quant_bytes(qtype, V, D), np.uint8)
    mlk.quantize(qtype, table, V, D, blocks)
    ids = W.zipf_ids(T, V, 1.1, cfg["seed"])
    ids[:2] = [0, V - 1]
    d_ids = mlk.DeviceBuffer.from_array(ids)
    out = mlk.DeviceBuffer.empty((T, D))
    mlk.gather_quant(qtype, blocks, V, D, d_ids, T, out)
    hblocks = blocks.download()
    got = out.download()
    assert_bits_equal(got, orc.gather_quant(qtype, hblocks, V, D, ids), f"{qtype} gather")
    # the device quantizer writes TensorToQ* bytes: check the rows that were
    # gathered plus a spread of others against the CPU quantizer
    rows = np.unique(np.concatenate([ids, np.arange(0, V, 997)]))
    bb = W.BLOCK_BYTES[qtype] * (D // 32)
    htable = table.download()
    np.testing.assert_array_equal(hblocks.reshape(V, bb)[rows],
                                  orc.quantize(qtype, htable[rows]).reshape(len(rows), bb))
    # quantization error is bounded by the block scale
    err = np.abs(got - htable[ids]).max()
    assert err < {"q8_0": 0.002, "q4_0": 0.02, "q4_1": 0.01}[qtype], err


@pytest.mark.parametrize("T", [1, 7, 64])
def test_decode_chain(mlk, orc, T):
    """Configs[1]: decode steps with positions uniform in [0, 8191]."""
    cfg = W.CONFIGS["c2_decode_8b"]
    V, D, H, KV, hd, F = (cfg[k] for k in ("vocab", "dim", "n_heads", "n_kv_heads", "head_dim",
                                           "ffn"))
    rng = np.random.default_rng(T)
    table = device_normal(mlk, (V, D), 0.0, 0.02, 99)
    ids = W.zipf_ids(T, V, 1.1, T)
    pos = W.decode_positions(T, cfg["max_pos"], T)
    delta = (rng.standard_normal((T, D)) * 0.02).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    q = (rng.standard_normal((T, H * hd)) * 0.02).astype(np.float32)
    k = (rng.standard_normal((T, KV * hd)) * 0.02).astype(np.float32)
    gate = (rng.standard_normal((T, F)) * 0.02).astype(np.float32)
    up = (rng.standard_normal((T, F)) * 0.02).astype(np.float32)
    d_x = mlk.DeviceBuffer.empty((T, D))
    d_y = mlk.DeviceBuffer.empty((T, D))
    d_ids, d_pos = mlk.DeviceBuffer.from_array(ids), mlk.DeviceBuffer.from_array(pos)
    d_delta, d_w = mlk.DeviceBuffer.from_array(delta), mlk.DeviceBuffer.from_array(w)
    d_q, d_k = mlk.DeviceBuffer.from_array(q), mlk.DeviceBuffer.from_array(k)
    d_g, d_u = mlk.DeviceBuffer.from_array(gate), mlk.DeviceBuffer.from_array(up)
    d_o = mlk.DeviceBuffer.empty((T, F))
    mlk.gather_f32(table, V, D, d_ids, T, d_x)
    mlk.add_rmsnorm(d_x, d_delta, d_w, d_y, T, D, cfg["eps"])
    mlk.rope(d_q, d_k, T, H, KV, hd, positions=d_pos, theta=cfg["theta"])
    mlk.swiglu(d_g, d_u, d_o, T * F)
    ex = orc.gather_f32(table.download(), ids)
    er, ey = orc.add_rmsnorm(ex, delta, w, cfg["eps"])
    assert_bits_equal(d_x.download(), er, "residual")
    assert_terms_close(d_y.download(), ey, np.abs(ey), "norm")
    eq, ek = orc.rope(q, k, H, KV, hd, positions=pos, theta=cfg["theta"])
    assert_terms_close(d_q.download(), eq, np.abs(eq), "q")
    assert_terms_close(d_k.download(), ek, np.abs(ek), "k")
    eo = orc.swiglu(gate, up)
    assert_terms_close(d_o.download(), eo, np.abs(eo), "ffn")


# ------------------------------------------------------------ linear (decode)

@pytest.mark.parametrize("qt,out_f,in_f,T", [
    ("q8_0", 14336, 4096, 1), ("q8_0", 4096, 14336, 4), ("q4_0", 14336, 4096, 1),
    ("q4_0", 4096, 14336, 2), ("q4_1", 14336, 4096, 4), ("q4_1", 6144, 4096, 1),
    ("q8_0", 128256, 4096, 1)])
def test_quant_linear_decode_full_size(mlk, orc, qt, out_f, in_f, T):
    """Llama-3-8B projections (gate/up [14336, 4096], down [4096, 14336],
    fused QKV [6144, 4096], lm_head [128256, 4096]) at decode batch sizes,
    weights quantized on the device from N(0, 0.02)."""
    w = device_normal(mlk, (out_f, in_f), 0.0, 0.02, out_f + in_f)
    blocks = mlk.DeviceBuffer(mlk.quant_bytes(qt, out_f, in_f), np.uint8)
    mlk.quantize(qt, w, out_f, in_f, blocks)
    del w
    x = device_normal(mlk, (T, in_f), 0.0, 1.0, 7 + T)
    y = mlk.DeviceBuffer.empty((T, out_f))
    mlk.linear_quant(qt, x, blocks, y, T, in_f, out_f)
    got = y.download()
    hb = blocks.download()
    del blocks
    ex, s = dot_exact(x.download(), orc.dequantize(qt, hb, out_f, in_f))
    assert_dot_close(got, ex, s, in_f, f"{qt} {out_f}x{in_f} T={T}")


def test_f32_linear_decode_full_size(mlk, orc):
    out_f, in_f, T = 14336, 4096, 2
    w = device_normal(mlk, (out_f, in_f), 0.0, 0.02, 3)
    x = device_normal(mlk, (T, in_f), 0.0, 1.0, 4)
    y = mlk.DeviceBuffer.empty((T, out_f))
    mlk.linear_f32(x, w, y, T, in_f, out_f)
    ex, s = dot_exact(x.download(), w.download())
    assert_dot_close(y.download(), ex, s, in_f, "f32 14336x4096")
