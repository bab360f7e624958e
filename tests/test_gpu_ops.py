"""GPU parity: every HIP op through the C ABI against the CPU oracle and the
reference's golden fixtures.

Bars (north star): gather and quantized gather bit-exact; residual add
bit-exact; RMSNorm / RoPE / SwiGLU within 1e-5 * max(1, sum|terms|)
(README.md:7, test/ops_test.cc:520-521).  Shapes cover the reference's own
test cases (test/cuda_ops_test.cc, tests/test_cuda_ops.cc) plus ragged and
unaligned widths.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_bits_equal, assert_terms_close, golden, max_ulp

pytestmark = pytest.mark.gpu


def normal(rng, shape, mean=0.0, std=1.0):
    return (rng.standard_normal(shape) * std + mean).astype(np.float32)


def values(shape):
    """test/cuda_ops_test.cc:70-76 input pattern."""
    n = int(np.prod(shape))
    return ((np.arange(n) % 29 - 14) / 7.0).astype(np.float32).reshape(shape)


# ------------------------------------------------------------- tiny chain

def test_tiny_chain_matches_reference_golden(mlk):
    g = golden("tiny_chain")
    T, D, H, KV, hd, F = len(g["ids"]), int(g["dim"]), int(g["n_heads"]), int(g["n_kv_heads"]), \
        int(g["head_dim"]), int(g["ffn_dim"])
    d_table = mlk.DeviceBuffer.from_array(g["table"])
    d_ids = mlk.DeviceBuffer.from_array(g["ids"])
    d_x = mlk.DeviceBuffer.empty((T, D))
    mlk.gather_f32(d_table, int(g["vocab"]), D, d_ids, T, d_x)
    assert_bits_equal(d_x.download(), g["gathered"], "gather")
    d_delta = mlk.DeviceBuffer.from_array(g["delta"])
    d_w = mlk.DeviceBuffer.from_array(g["norm_w"])
    d_y = mlk.DeviceBuffer.empty((T, D))
    mlk.add_rmsnorm(d_x, d_delta, d_w, d_y, T, D, float(g["eps"]))
    assert_bits_equal(d_x.download(), g["residual_out"], "residual")
    y = d_y.download()
    assert_terms_close(y, g["norm_out"], np.abs(g["norm_out"]), "rmsnorm")
    d_q = mlk.DeviceBuffer.from_array(g["q"])
    d_k = mlk.DeviceBuffer.from_array(g["k"])
    d_pos = mlk.DeviceBuffer.from_array(g["positions"])
    mlk.rope(d_q, d_k, T, H, KV, hd, positions=d_pos, theta=float(g["theta"]))
    assert_terms_close(d_q.download(), g["q_out"], np.abs(g["q_out"]), "rope q")
    assert_terms_close(d_k.download(), g["k_out"], np.abs(g["k_out"]), "rope k")
    d_g = mlk.DeviceBuffer.from_array(g["gate"])
    d_u = mlk.DeviceBuffer.from_array(g["up"])
    d_o = mlk.DeviceBuffer.empty((T, F))
    mlk.swiglu(d_g, d_u, d_o, T * F)
    assert_terms_close(d_o.download(), g["ffn_out"], np.abs(g["ffn_out"]), "swiglu")


# ---------------------------------------------------------------- rmsnorm

@pytest.mark.parametrize("rows,dim", [(1, 1), (1, 7), (1, 86), (3, 259), (2, 1025), (5, 4096),
                                      (3, 4100), (2, 8192), (1, 16384), (2, 20000), (64, 4096)])
def test_add_rmsnorm_matches_oracle(mlk, orc, rows, dim):
    rng = np.random.default_rng(rows * 100003 + dim)
    x = normal(rng, (rows, dim), std=0.02)
    d = normal(rng, (rows, dim), std=0.02)
    w = normal(rng, (dim,), mean=1.0, std=0.1)
    exp_r, exp_y = orc.add_rmsnorm(x, d, w, 1e-5)
    d_x = mlk.DeviceBuffer.from_array(x)
    d_d = mlk.DeviceBuffer.from_array(d)
    d_w = mlk.DeviceBuffer.from_array(w)
    d_y = mlk.DeviceBuffer.empty((rows, dim))
    mlk.add_rmsnorm(d_x, d_d, d_w, d_y, rows, dim, 1e-5)
    assert_bits_equal(d_x.download(), exp_r, "residual")
    y = d_y.download()
    assert_terms_close(y, exp_y, np.abs(exp_y), "y")
    print(f"rmsnorm [{rows},{dim}] max ulp vs oracle: {max_ulp(y, exp_y)}")


@pytest.mark.parametrize("n", [1, 7, 259, 1025])
@pytest.mark.parametrize("zero", [False, True])
def test_rmsnorm_reference_cases(mlk, orc, n, zero):
    """test/cuda_ops_test.cc:105-126: sizes 1, 7, 259, 1025, zero input; the
    input is not modified."""
    x = values((n,))
    if zero:
        x[:] = 0
    w = values((n,))
    exp = orc.rmsnorm(x, w, 1e-5)
    d_x = mlk.DeviceBuffer.from_array(x)
    d_w = mlk.DeviceBuffer.from_array(w)
    d_y = mlk.DeviceBuffer.empty((n,))
    mlk.rmsnorm(d_x, d_w, d_y, 1, n, 1e-5)
    assert_terms_close(d_y.download(), exp, np.abs(exp), "rmsnorm")
    assert_bits_equal(d_x.download(), x, "input untouched")


def test_rmsnorm_golden_rows(mlk):
    g = golden("rows_8b_70b")
    for tag in ("8b", "70b"):
        x, w, y = g[f"rms_{tag}_x"], g[f"rms_{tag}_w"], g[f"rms_{tag}_y"]
        d_x = mlk.DeviceBuffer.from_array(x)
        d_w = mlk.DeviceBuffer.from_array(w)
        d_y = mlk.DeviceBuffer.empty(x.shape)
        mlk.rmsnorm(d_x, d_w, d_y, 1, x.size, 1e-5)
        assert_terms_close(d_y.download(), y, np.abs(y), f"rmsnorm {tag}")


def test_rmsnorm_in_place_and_unaligned(mlk, orc):
    rng = np.random.default_rng(5)
    x = normal(rng, (4, 257))
    w = normal(rng, (257,), mean=1.0, std=0.1)
    exp = orc.rmsnorm(x, w, 1e-5)
    buf = mlk.DeviceBuffer(x.nbytes + 4)
    mlk.lib.mlk_memcpy(buf.ptr + 4, x.ctypes.data, x.nbytes, mlk.H2D)
    d_w = mlk.DeviceBuffer.from_array(w)
    mlk.rmsnorm(buf.ptr + 4, d_w, buf.ptr + 4, 4, 257, 1e-5)  # in place, 4-byte aligned
    out = np.empty_like(x)
    mlk.check(mlk.lib.mlk_memcpy(out.ctypes.data, buf.ptr + 4, x.nbytes, mlk.D2H))
    assert_terms_close(out, exp, np.abs(exp), "in-place unaligned")


# ----------------------------------------------------------------- swiglu

@pytest.mark.parametrize("n", [1, 3, 4, 5, 173, 1024, 1027, 14336 * 3 + 1, 1 << 20])
def test_swiglu_and_parts_match_oracle(mlk, orc, n):
    rng = np.random.default_rng(n)
    g = normal(rng, (n,), std=2.0)
    u = normal(rng, (n,))
    d_g = mlk.DeviceBuffer.from_array(g)
    d_u = mlk.DeviceBuffer.from_array(u)
    d_y = mlk.DeviceBuffer.empty((n,))
    mlk.swiglu(d_g, d_u, d_y, n)
    exp = orc.swiglu(g, u)
    y = d_y.download()
    assert_terms_close(y, exp, np.abs(exp), "swiglu")
    mlk.silu(d_g, d_y, n)
    exp_s = orc.silu(g)
    assert_terms_close(d_y.download(), exp_s, np.abs(exp_s), "silu")
    mlk.mul(d_g, d_u, d_y, n)
    assert_bits_equal(d_y.download(), orc.mul(g, u), "mul")
    mlk.add(d_g, d_u, d_y, n)
    assert_bits_equal(d_y.download(), orc.add(g, u), "add")
    print(f"swiglu n={n} max ulp vs oracle: {max_ulp(y, exp)}")


def test_swiglu_golden_rows(mlk):
    g = golden("rows_8b_70b")
    for tag in ("8b", "70b"):
        gate, up, y = g[f"swiglu_{tag}_g"], g[f"swiglu_{tag}_u"], g[f"swiglu_{tag}_y"]
        d_g = mlk.DeviceBuffer.from_array(gate)
        d_u = mlk.DeviceBuffer.from_array(up)
        d_y = mlk.DeviceBuffer.empty(gate.shape)
        mlk.swiglu(d_g, d_u, d_y, gate.size)
        assert_terms_close(d_y.download(), y, np.abs(y), f"swiglu {tag}")
        x, sy = g[f"silu_{tag}_x"], g[f"silu_{tag}_y"]
        d_x = mlk.DeviceBuffer.from_array(x)
        d_sy = mlk.DeviceBuffer.empty(x.shape)
        mlk.silu(d_x, d_sy, x.size)
        assert_terms_close(d_sy.download(), sy, np.abs(sy), f"silu {tag}")


def test_swiglu_unaligned_pointers(mlk, orc):
    rng = np.random.default_rng(9)
    n = 1001
    g = normal(rng, (n,))
    u = normal(rng, (n,))
    big = mlk.DeviceBuffer(4 * (3 * n + 3))
    pg, pu, py = big.ptr + 4, big.ptr + 4 * (n + 2), big.ptr + 4 * (2 * n + 3)
    mlk.check(mlk.lib.mlk_memcpy(pg, g.ctypes.data, g.nbytes, mlk.H2D))
    mlk.check(mlk.lib.mlk_memcpy(pu, u.ctypes.data, u.nbytes, mlk.H2D))
    mlk.swiglu(pg, pu, py, n)
    out = np.empty(n, np.float32)
    mlk.check(mlk.lib.mlk_memcpy(out.ctypes.data, py, out.nbytes, mlk.D2H))
    exp = orc.swiglu(g, u)
    assert_terms_close(out, exp, np.abs(exp), "unaligned swiglu")


# ------------------------------------------------------------------- rope

ROPE_CASES = [
    # (T, H, KV, hd, theta)
    (1, 4, 2, 8, 10000.0),      # tests/test_cuda_ops.cc:32-48
    (1, 5, 2, 2, 10000.0),      # test/cuda_ops_test.cc:185-210 (head_dim 2, 8, 130)
    (1, 5, 2, 8, 10000.0),
    (1, 5, 2, 130, 10000.0),
    (6, 4, 2, 16, 10000.0),     # tiny config
    (7, 32, 8, 128, 500000.0),  # 8B decode-like
    (3, 64, 8, 128, 500000.0),  # 70B
    (2, 3, 1, 6, 100.0),
    (2, 128, 128, 128, 10000.0),  # too many heads for one batch per lane: general kernel
]


@pytest.mark.parametrize("rope_type", [0, 1])
@pytest.mark.parametrize("T,H,KV,hd,theta", ROPE_CASES)
def test_rope_matches_oracle(mlk, orc, T, H, KV, hd, theta, rope_type):
    rng = np.random.default_rng(T * 1000 + H * 10 + hd)
    q = normal(rng, (T, H * hd))
    k = normal(rng, (T, KV * hd), std=0.3)
    pos = rng.integers(0, 8192, size=T).astype(np.int32)
    pos[0] = 0
    exp_q, exp_k = orc.rope(q, k, H, KV, hd, positions=pos, theta=theta, rope_type=rope_type)
    d_q = mlk.DeviceBuffer.from_array(q)
    d_k = mlk.DeviceBuffer.from_array(k)
    d_pos = mlk.DeviceBuffer.from_array(pos)
    mlk.rope(d_q, d_k, T, H, KV, hd, positions=d_pos, theta=theta, rope_type=rope_type)
    gq, gk = d_q.download(), d_k.download()
    assert_terms_close(gq, exp_q, np.abs(exp_q), "q")
    assert_terms_close(gk, exp_k, np.abs(exp_k), "k")
    # contiguous positions from pos0 (the reference's one-token signature is T = 1)
    d_q.upload(q)
    d_k.upload(k)
    mlk.rope(d_q, d_k, T, H, KV, hd, pos0=7, theta=theta, rope_type=rope_type)
    eq, ek = orc.rope(q, k, H, KV, hd, pos0=7, theta=theta, rope_type=rope_type)
    assert_terms_close(d_q.download(), eq, np.abs(eq), "q pos0")
    assert_terms_close(d_k.download(), ek, np.abs(ek), "k pos0")
    print(f"rope T={T} H={H} KV={KV} hd={hd} type={rope_type} max ulp: "
          f"{max(max_ulp(gq, exp_q), max_ulp(gk, exp_k))}")


# Workgroups walk tokens t = block + j * grid, two per loop trip with the
# last one or two peeled: token counts that leave every workgroup 1..5
# tokens (grid: 1024 resident threads per CU in workgroups of 256 threads at
# 8B heads, 512 at 70B, 64 for the small heads).
@pytest.mark.parametrize("rope_type", [0, 1])
@pytest.mark.parametrize("per_cu,H,KV,hd", [(4, 32, 8, 128), (16, 4, 2, 16), (16, 14, 2, 64),
                                            (2, 64, 8, 128)])
@pytest.mark.parametrize("trips", [1, 2, 3, 4])
def test_rope_tokens_per_workgroup(mlk, orc, trips, per_cu, H, KV, hd, rope_type):
    grid = per_cu * mlk.device_info()["compute_units"]
    T = trips * grid + 2 * trips + 1  # the first workgroups get one token more
    rng = np.random.default_rng(trips * 7 + H + rope_type)
    q = normal(rng, (T, H * hd))
    k = normal(rng, (T, KV * hd), std=0.3)
    pos = rng.integers(0, 8192, size=T).astype(np.int32)
    exp_q, exp_k = orc.rope(q, k, H, KV, hd, positions=pos, theta=500000.0, rope_type=rope_type)
    d_q = mlk.DeviceBuffer.from_array(q)
    d_k = mlk.DeviceBuffer.from_array(k)
    d_pos = mlk.DeviceBuffer.from_array(pos)
    mlk.rope(d_q, d_k, T, H, KV, hd, positions=d_pos, theta=500000.0, rope_type=rope_type)
    assert_terms_close(d_q.download(), exp_q, np.abs(exp_q), f"q T={T}")
    assert_terms_close(d_k.download(), exp_k, np.abs(exp_k), f"k T={T}")


def test_rope_golden_positions(mlk):
    """Reference outputs at pos 0, 1, 4095, 8191, theta 5e5, 8B heads."""
    g = golden("rows_8b_70b")
    for pos in (0, 1, 4095, 8191):
        for rt, name in ((0, "normal"), (1, "neox")):
            d_q = mlk.DeviceBuffer.from_array(g[f"rope_p{pos}_q"])
            d_k = mlk.DeviceBuffer.from_array(g[f"rope_p{pos}_k"])
            mlk.rope(d_q, d_k, 1, 32, 8, 128, pos0=pos, theta=500000.0, rope_type=rt)
            eq, ek = g[f"rope_p{pos}_{name}_q"], g[f"rope_p{pos}_{name}_k"]
            assert_terms_close(d_q.download(), eq, np.abs(eq), f"q pos {pos} {name}")
            assert_terms_close(d_k.download(), ek, np.abs(ek), f"k pos {pos} {name}")
            if pos == 0:
                assert_bits_equal(d_q.download(), g[f"rope_p{pos}_q"], "pos 0 is identity")


def test_rope_reference_kat(mlk):
    """test/ops_test.cc:749-769: pos 1, theta 100, one head of width 4."""
    q = np.array([1, 2, 3, 4], np.float32)
    k = np.array([-2, 0.5, 1, -3], np.float32)
    want = {0: ([-1.1426396637476532, 1.922075596544176, 2.585678829246765, 4.279516911052588],
                [-1.501340104140228, -1.4127908166817231, 1.2945044152185103,
                 -2.8851790791872496]),
            1: ([-1.9841106485555495, 1.590674663968739, 2.4623779024123156, 4.17968349440576],
                [-1.922075596544176, 0.7970023325794974, -1.1426396637476532,
                 -2.9350957875106634])}
    for rt, (wq, wk) in want.items():
        d_q = mlk.DeviceBuffer.from_array(q)
        d_k = mlk.DeviceBuffer.from_array(k)
        mlk.rope(d_q, d_k, 1, 1, 1, 4, pos0=1, theta=100.0, rope_type=rt)
        np.testing.assert_allclose(d_q.download(), wq, rtol=0, atol=2e-5 * max(1, 4.3))
        np.testing.assert_allclose(d_k.download(), wk, rtol=0, atol=2e-5 * max(1, 3.0))


def test_rope_strided_fused_qkv(mlk, orc):
    """q and k as column slices of a fused [T, (H + 2 KV) * hd] activation."""
    rng = np.random.default_rng(3)
    T, H, KV, hd = 5, 8, 2, 64
    width = (H + 2 * KV) * hd
    qkv = normal(rng, (T, width))
    pos = np.array([0, 3, 100, 4095, 8191], np.int32)
    d = mlk.DeviceBuffer.from_array(qkv)
    d_pos = mlk.DeviceBuffer.from_array(pos)
    mlk.rope(d.ptr, d.ptr + 4 * H * hd, T, H, KV, hd, positions=d_pos, theta=500000.0,
             q_row_stride=width, k_row_stride=width)
    out = d.download()
    eq, ek = orc.rope(qkv[:, :H * hd], qkv[:, H * hd:(H + KV) * hd], H, KV, hd, positions=pos,
                      theta=500000.0)
    assert_terms_close(out[:, :H * hd], eq, np.abs(eq), "q slice")
    assert_terms_close(out[:, H * hd:(H + KV) * hd], ek, np.abs(ek), "k slice")
    assert_bits_equal(out[:, (H + KV) * hd:], qkv[:, (H + KV) * hd:], "v untouched")


def test_rope_negative_position_flags_and_skips(mlk, orc):
    rng = np.random.default_rng(4)
    q = normal(rng, (3, 2 * 8))
    k = normal(rng, (3, 1 * 8))
    pos = np.array([2, -1, 5], np.int32)
    d_q = mlk.DeviceBuffer.from_array(q)
    d_k = mlk.DeviceBuffer.from_array(k)
    d_pos = mlk.DeviceBuffer.from_array(pos)
    err = mlk.DeviceBuffer.from_array(np.zeros(1, np.int32))
    mlk.rope(d_q, d_k, 3, 2, 1, 8, positions=d_pos, err=err)
    assert err.download()[0] != 0
    gq = d_q.download()
    assert_bits_equal(gq[1], q[1], "negative-position token untouched")
    eq, _ = orc.rope(q[[0, 2]], k[[0, 2]], 2, 1, 8, positions=pos[[0, 2]])
    assert_terms_close(gq[[0, 2]], eq, np.abs(eq), "other tokens rotated")


# ----------------------------------------------------------------- gather

@pytest.mark.parametrize("vocab,dim", [(3, 259), (131, 64), (131, 32), (7, 5), (1000, 4096)])
def test_gather_f32_bit_exact(mlk, orc, vocab, dim):
    rng = np.random.default_rng(vocab + dim)
    table = normal(rng, (vocab, dim), std=0.02)
    ids = np.array([0, vocab - 1, 1 % vocab] + list(rng.integers(0, vocab, 29)), np.int32)
    d_t = mlk.DeviceBuffer.from_array(table)
    d_ids = mlk.DeviceBuffer.from_array(ids)
    d_o = mlk.DeviceBuffer.empty((len(ids), dim))
    mlk.gather_f32(d_t, vocab, dim, d_ids, len(ids), d_o)
    assert_bits_equal(d_o.download(), orc.gather_f32(table, ids), "gather")
    for token in (0, vocab - 1):  # one-token host id (CudaEmbeddingDevice)
        d_one = mlk.DeviceBuffer.empty((1, dim))
        mlk.gather_f32(d_t, vocab, dim, None, 1, d_one, token=token)
        assert_bits_equal(d_one.download()[0], table[token], f"token {token}")


def test_gather_f32_invalid_ids_flag_zero_rows(mlk):
    table = values((4, 12))
    ids = np.array([1, 4, -1, 3], np.int32)
    d_t = mlk.DeviceBuffer.from_array(table)
    d_ids = mlk.DeviceBuffer.from_array(ids)
    d_o = mlk.DeviceBuffer.empty((4, 12))
    err = mlk.DeviceBuffer.from_array(np.zeros(1, np.int32))
    mlk.gather_f32(d_t, 4, 12, d_ids, 4, d_o, err=err)
    out = d_o.download()
    assert err.download()[0] != 0
    assert_bits_equal(out[[0, 3]], table[[1, 3]], "valid rows")
    assert (out[[1, 2]] == 0).all()
    for qt in ("q8_0", "q4_0", "q4_1"):
        blocks = mlk.DeviceBuffer(mlk.quant_bytes(qt, 4, 12), np.uint8)
        mlk.quantize(qt, d_t, 4, 12, blocks)
        err.upload(np.zeros(1, np.int32))
        mlk.gather_quant(qt, blocks, 4, 12, d_ids, 4, d_o, err=err)
        assert err.download()[0] != 0
        assert (d_o.download()[[1, 2]] == 0).all()


@pytest.mark.parametrize("qtype", ["q8_0", "q4_0", "q4_1"])
@pytest.mark.parametrize("vocab,dim", [(5, 7), (9, 33), (11, 100), (131, 64), (64, 4096),
                                       (17, 8192), (3, 4100)])
def test_quantize_and_gather_quant_bit_exact(mlk, orc, qtype, vocab, dim):
    rng = np.random.default_rng(vocab * 7 + dim)
    table = normal(rng, (vocab, dim), std=0.02)
    d_t = mlk.DeviceBuffer.from_array(table)
    nbytes = mlk.quant_bytes(qtype, vocab, dim)
    d_b = mlk.DeviceBuffer(nbytes, np.uint8)
    mlk.quantize(qtype, d_t, vocab, dim, d_b)
    blocks = d_b.download()
    np.testing.assert_array_equal(blocks, orc.quantize(qtype, table), "device quantizer")
    ids = np.array([0, vocab - 1] + list(rng.integers(0, vocab, 40)), np.int32)
    d_ids = mlk.DeviceBuffer.from_array(ids)
    d_o = mlk.DeviceBuffer.empty((len(ids), dim))
    mlk.gather_quant(qtype, d_b, vocab, dim, d_ids, len(ids), d_o)
    assert_bits_equal(d_o.download(), orc.gather_quant(qtype, blocks, vocab, dim, ids), qtype)
    d_one = mlk.DeviceBuffer.empty((1, dim))
    mlk.gather_quant(qtype, d_b, vocab, dim, None, 1, d_one, token=vocab - 1)
    assert_bits_equal(d_one.download()[0], orc.dequantize(qtype, blocks, vocab, dim)[-1], "one")


@pytest.mark.parametrize("qtype", ["q8_0", "q4_0", "q4_1"])
def test_gather_quant_golden_blocks(mlk, qtype):
    """Blocks and dequantized rows written by the reference: C4-distribution
    rows, ragged widths, edge rows, hand-made scales (0, subnormal 0x0001,
    0x3400, 0x3A00, 0x4000) and Q4_1 minima."""
    q = golden("quant")
    for name in ("c4", "ragged100", "ragged33", "ragged7", "edge"):
        x = q[f"{name}_x"]
        rows, cols = x.shape
        blocks = q[f"{name}_{qtype}_blocks"]
        d_x = mlk.DeviceBuffer.from_array(x)
        d_b = mlk.DeviceBuffer(mlk.quant_bytes(qtype, rows, cols), np.uint8)
        mlk.quantize(qtype, d_x, rows, cols, d_b)
        np.testing.assert_array_equal(d_b.download(), blocks, f"{name} blocks")
        ids = np.arange(rows, dtype=np.int32)[::-1].copy()
        d_b.upload(blocks)
        d_ids = mlk.DeviceBuffer.from_array(ids)
        d_o = mlk.DeviceBuffer.empty((rows, cols))
        mlk.gather_quant(qtype, d_b, rows, cols, d_ids, rows, d_o)
        assert_bits_equal(d_o.download(), q[f"{name}_{qtype}_deq"][ids], f"{name} rows")
    k = golden("dequant_kat")
    rows, cols = int(k["rows"]), int(k["cols"])
    d_b = mlk.DeviceBuffer.from_array(k[f"{qtype}_blocks"])
    ids = np.arange(rows, dtype=np.int32)
    d_ids = mlk.DeviceBuffer.from_array(ids)
    d_o = mlk.DeviceBuffer.empty((rows, cols))
    mlk.gather_quant(qtype, d_b, rows, cols, d_ids, rows, d_o)
    assert_bits_equal(d_o.download(), k[f"{qtype}_deq"], "handcrafted blocks")
    assert_bits_equal(d_o.download(), k[f"{qtype}_deq_flat"], "QuanTensor overload")


@pytest.mark.parametrize("qtype", ["q8_0", "q4_0", "q4_1"])
def test_gather_quant_special_scales(mlk, orc, qtype):
    """fp16 scales that are subnormal, inf and NaN (payload kept) decode like
    the CPU Fp16ToFp32."""
    bb = {"q8_0": 34, "q4_0": 18, "q4_1": 20}[qtype]
    codes = [0x0001, 0x03FF, 0x0400, 0x7BFF, 0x7C00, 0xFC00, 0x7C01, 0x7E00, 0x8001, 0x3C00]
    rng = np.random.default_rng(1)
    raw = rng.integers(0, 256, size=(len(codes), bb), dtype=np.uint8)
    for i, c in enumerate(codes):
        raw[i, 0:2] = [c & 0xFF, c >> 8]
        if qtype == "q4_1":
            m = codes[(i + 3) % len(codes)]
            raw[i, 2:4] = [m & 0xFF, m >> 8]
    blocks = raw.reshape(-1).copy()
    vocab, dim = len(codes), 32
    d_b = mlk.DeviceBuffer.from_array(blocks)
    ids = np.arange(vocab, dtype=np.int32)
    d_ids = mlk.DeviceBuffer.from_array(ids)
    d_o = mlk.DeviceBuffer.empty((vocab, dim))
    mlk.gather_quant(qtype, d_b, vocab, dim, d_ids, vocab, d_o)
    # NaN results compare as NaN: the default NaN of an invalid product
    # (inf * 0) is platform-specific, while decoded NaN payloads are kept.
    assert_bits_equal(d_o.download(), orc.gather_quant(qtype, blocks, vocab, dim, ids), "special",
                      nan_equal=True)


# ---------------------------------------------------------------- softmax

def test_softmax_reference_cases(mlk, orc):
    """test/cuda_ops_test.cc:155-183 and the golden rows."""
    g = golden("rows_8b_70b")
    cases = [np.array(v, np.float32) for v in ([3.0], [2.0, 2.0, 2.0], [-5.0, -2.0, -9.0],
                                               [10000.0, 10001.0, -10000.0])]
    cases += [values((259,)), values((1025,)), g["softmax_x"], g["softmax_big_x"]]
    for x in cases:
        d_x = mlk.DeviceBuffer.from_array(x)
        d_y = mlk.DeviceBuffer.empty(x.shape)
        mlk.softmax(d_x, d_y, 1, x.size)
        y = d_y.download()
        m = np.max(x.astype(np.float64))
        e = np.exp(x.astype(np.float64) - m)
        exact = e / e.sum()
        np.testing.assert_allclose(y, exact, rtol=0, atol=1e-5 * (1 + np.abs(exact)).max())
        assert abs(float(y.astype(np.float64).sum()) - 1.0) < 1e-5
    assert_terms_close(
        _softmax_dev(mlk, g["softmax_x"]), g["softmax_y"], np.abs(g["softmax_y"]), "golden")


def _softmax_dev(mlk, x):
    d_x = mlk.DeviceBuffer.from_array(x)
    d_y = mlk.DeviceBuffer.empty(x.shape)
    mlk.softmax(d_x, d_y, 1, x.size)
    return d_y.download()


# --------------------------------------------------------- rejected input

def test_invalid_arguments_are_rejected_before_launch(mlk):
    d = mlk.DeviceBuffer.from_array(values((4, 4)))
    w = mlk.DeviceBuffer.from_array(values((4,)))
    y = mlk.DeviceBuffer.empty((4, 4))
    for eps in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(mlk.MlkError, match="eps must be finite and positive"):
            mlk.add_rmsnorm(d, None, w, y, 4, 4, eps)
    with pytest.raises(mlk.MlkError, match="must not be null"):
        mlk.rmsnorm(d, None, y, 4, 4, 1e-5)
    with pytest.raises(mlk.MlkError, match="alias"):
        mlk.add_rmsnorm(d, w, w, d, 4, 4, 1e-5)
    with pytest.raises(mlk.MlkError, match="must not be empty"):
        mlk.swiglu(d, d, y, 0)
    for theta in (0.0, -1.0, float("inf"), float("nan")):
        with pytest.raises(mlk.MlkError, match="theta must be finite and positive"):
            mlk.rope(d, w, 1, 2, 1, 4, pos0=0, theta=theta)
    with pytest.raises(mlk.MlkError, match="pos must be non-negative"):
        mlk.rope(d, w, 1, 2, 1, 4, pos0=-1)
    for H, KV, hd in ((0, 1, 4), (2, 0, 4), (2, 1, 0), (2, 1, 3)):
        with pytest.raises(mlk.MlkError, match="head_dim must be positive and even"):
            mlk.rope(d, w, 1, H, KV, hd, pos0=0)
    with pytest.raises(mlk.MlkError, match="token_id must be in"):
        mlk.gather_f32(d, 4, 4, None, 1, y, token=4)
    with pytest.raises(mlk.MlkError, match="token_id must be in"):
        mlk.gather_f32(d, 4, 4, None, 1, y, token=-1)
    with pytest.raises(mlk.MlkError, match="weight dimensions must be positive"):
        mlk.gather_f32(d, 0, 4, None, 1, y, token=0)
    with pytest.raises(mlk.MlkError, match="must not be null"):
        mlk.gather_f32(None, 4, 4, None, 1, y, token=0)
    # nothing above touched the output
    mlk.synchronize()


def test_empty_batches_are_no_ops(mlk):
    d = mlk.DeviceBuffer.from_array(values((2, 8)))
    mlk.rope(d, d, 0, 1, 1, 8, pos0=0)
    mlk.gather_f32(d, 2, 8, d, 0, None)
    assert_bits_equal(d.download(), values((2, 8)), "unchanged")


@pytest.mark.parametrize("qtype", ["q8_0", "q4_0", "q4_1"])
@pytest.mark.parametrize("offset", [1, 2, 4])
def test_gather_quant_unaligned_table(mlk, orc, qtype, offset):
    """A table that starts 1, 2 or 4 bytes into an allocation (odd offsets
    force the byte-load path, 2 keeps u16 words aligned but not the Q4_1 u32
    words)."""
    rng = np.random.default_rng(offset)
    vocab, dim = 7, 96
    table = normal(rng, (vocab, dim), std=0.5)
    blocks = orc.quantize(qtype, table)
    buf = mlk.DeviceBuffer(blocks.nbytes + 16, np.uint8)
    mlk.check(mlk.lib.mlk_memcpy(buf.ptr + offset, blocks.ctypes.data, blocks.nbytes, mlk.H2D))
    ids = np.array([6, 0, 3, 3, 1], np.int32)
    d_ids = mlk.DeviceBuffer.from_array(ids)
    d_o = mlk.DeviceBuffer.empty((len(ids), dim))
    mlk.gather_quant(qtype, buf.ptr + offset, vocab, dim, d_ids, len(ids), d_o)
    assert_bits_equal(d_o.download(), orc.gather_quant(qtype, blocks, vocab, dim, ids), "unaligned")
