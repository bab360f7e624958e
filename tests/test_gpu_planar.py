"""The planar weight layout (mlk_quant_to_planar) and the linear layers over
it (mlk_linear_planar): up to 32 rows on the bf16 matrix cores with exact
products, more rows on the fp32 matrix-core GEMM.  The planar layout has no
counterpart in the reference; its values are the reference blocks' (the
same scale and codes per element), so the results are held to the bar of
the block-layout linear layers: within gamma_K * sum|x w| of the exact
float64 value (tests/conftest.py:assert_dot_close), against the oracle's
dequantization of the same blocks (src/quant.cc:369-463)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_dot_close, dot_exact

pytestmark = pytest.mark.gpu

QT = ("q8_0", "q4_0")
BLOCK = {"q8_0": 34, "q4_0": 18}


def normal(rng, shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def planar_layout(qt, blocks, rows, cols):
    """The planar bytes of [rows, cols] blocks, from the format's statement
    (include/minilamma_hip.h, mlk_quant_to_planar)."""
    nb, bb = cols // 32, BLOCK[qt]
    blk = np.asarray(blocks, np.uint8).reshape(rows, nb, bb)
    tiles = (rows + 15) // 16
    pad = np.zeros((tiles * 16, nb, bb), np.uint8)
    pad[:rows] = blk
    scales = pad[:, :, 0:2].copy().view("<u2")[..., 0]          # [rows16, nb]
    if qt == "q8_0":
        codes = pad[:, :, 2:].reshape(tiles, 16, nb // 2, 2, 4, 8)  # t r pair j g e
        lanes = codes.transpose(0, 2, 4, 1, 3, 5)                   # t pair g r j e
        code_bytes = lanes.reshape(-1)
    else:
        qs = pad[:, :, 2:]
        nib = np.concatenate([qs & 15, qs >> 4], axis=2).astype(np.uint8) ^ 8  # [rows16, nb, 32]
        nib = nib.reshape(tiles, 16, nb // 4, 4, 4, 8)              # t r quad j g input
        lo, hi = nib[..., :4], nib[..., 4:]
        byte = (lo | (hi << 4)).astype(np.uint8)                    # t r quad j g e
        byte.reshape(tiles * 16, -1)[rows:] = 0                     # padding rows: zero bytes
        code_bytes = byte.transpose(0, 2, 4, 1, 3, 5).reshape(-1)   # t quad g r j e
    sc = scales.reshape(tiles, 16, nb // 8, 8).transpose(0, 2, 1, 3)  # t grp r e
    return np.concatenate([code_bytes, sc.astype("<u2").reshape(-1).view(np.uint8)])


def to_planar(mlk, qt, blocks, rows, cols):
    d_b = mlk.DeviceBuffer.from_array(np.ascontiguousarray(blocks, np.uint8))
    n = mlk.quant_planar_bytes(qt, rows, cols)
    assert n > 0
    d_p = mlk.DeviceBuffer(n, np.uint8)
    mlk.quant_to_planar(qt, d_b, rows, cols, d_p)
    return d_p


def run_planar(mlk, qt, x, planar, out_f, bias=None, workspace="auto"):
    x = np.atleast_2d(np.ascontiguousarray(x, np.float32))
    T, K = x.shape
    d_x = mlk.DeviceBuffer.from_array(x)
    d_bias = None if bias is None else mlk.DeviceBuffer.from_array(np.asarray(bias, np.float32))
    d_y = mlk.DeviceBuffer.empty((T, out_f))
    mlk.linear_planar(qt, d_x, planar, d_y, T, K, out_f, bias=d_bias, workspace=workspace)
    return d_y.download()


@pytest.mark.parametrize("qt", QT)
@pytest.mark.parametrize("rows,cols", [(16, 256), (37, 512), (130, 1024), (4099, 256)])
def test_planar_layout_bytes(mlk, orc, qt, rows, cols):
    """The repack writes exactly the stated layout (zero rows padding the
    last tile), for blocks with random codes and scales."""
    rng = np.random.default_rng(rows + cols)
    blocks = orc.quantize(qt, normal(rng, (rows, cols), 0.02))
    got = to_planar(mlk, qt, blocks, rows, cols).download()
    want = planar_layout(qt, blocks, rows, cols)
    assert got.size == want.size == mlk.quant_planar_bytes(qt, rows, cols)
    np.testing.assert_array_equal(got, want)


PLANAR_SHAPES = [  # (out, in, rows): one row takes the streaming GEMV (in_features up to
    # 14336; 1, 2, 4 or 8 chunks of 256 inputs per wave, idle waves, partial
    # tiles), 2..32 rows the bf16 kernel (one row too past 14336), more the GEMM
    (131, 256, 1), (4099, 4096, 1), (4096, 14336, 1), (300, 2816, 1), (1000, 11008, 1),
    (8192, 8192, 1), (17, 14592, 1),
    (64, 512, 3), (4096, 4096, 7), (100, 256, 16),
    (4097, 512, 17), (64, 4096, 31), (14336, 4096, 32), (4096, 14336, 12), (130, 768, 25),
    (1024, 4096, 33), (257, 512, 64), (200, 1024, 130)]


@pytest.mark.parametrize("qt", QT)
@pytest.mark.parametrize("shape", PLANAR_SHAPES)
def test_planar_linear_shapes(mlk, orc, qt, shape):
    """Token counts 1..32 (one and two 16-token tiles, partial tiles),
    output counts that end inside a 16-row tile or a 128-row workgroup, one
    to 57 K ranges; 33+ rows on the tiled GEMM (partial 128 x 128 tiles,
    split K); with a bias."""
    O, K, T = shape
    rng = np.random.default_rng(O + 7 * K + T)
    w = normal(rng, (O, K), 0.02)
    x = normal(rng, (T, K))
    bias = normal(rng, (O,), 0.1)
    blocks = orc.quantize(qt, w)
    ex, s = dot_exact(x, orc.dequantize(qt, blocks, O, K), bias)
    planar = to_planar(mlk, qt, blocks, O, K)
    got = run_planar(mlk, qt, x, planar, O, bias=bias)
    assert_dot_close(got, ex, s, K + 1, f"{qt} {shape}")


@pytest.mark.parametrize("qt", QT)
def test_planar_equals_block_layout_bound(mlk, orc, qt):
    """The planar and the block-layout kernels on the same blocks: both
    within the bound of the exact sums, at the 8B down projection's shape
    with 16 tokens (the batched decode step)."""
    O, K, T = 4096, 14336, 16
    rng = np.random.default_rng(11)
    blocks = orc.quantize(qt, normal(rng, (O, K), 0.02))
    x = normal(rng, (T, K))
    ex, s = dot_exact(x, orc.dequantize(qt, blocks, O, K))
    got_p = run_planar(mlk, qt, x, to_planar(mlk, qt, blocks, O, K), O)
    d_x, d_w = mlk.DeviceBuffer.from_array(x), mlk.DeviceBuffer.from_array(blocks)
    d_y = mlk.DeviceBuffer.empty((T, O))
    mlk.linear_quant(qt, d_x, d_w, d_y, T, K, O)
    assert_dot_close(got_p, ex, s, K, f"{qt} planar")
    assert_dot_close(d_y.download(), ex, s, K, f"{qt} blocks")


@pytest.mark.parametrize("qt", QT)
def test_planar_non_finite_inputs(mlk, orc, qt):
    """x with inf and NaN: every output whose sum meets them is what fp32
    products give (NaN, or inf of the sign the products force), the rest
    finite and within the bound; four rows (bf16 kernel) and each row alone
    (the one-row GEMV)."""
    O, K, T = 64, 512, 4
    rng = np.random.default_rng(3)
    blocks = orc.quantize(qt, normal(rng, (O, K), 0.02))
    wd = orc.dequantize(qt, blocks, O, K)
    x = normal(rng, (T, K))
    x[1, 5] = np.inf
    x[2, 300] = np.nan
    planar = to_planar(mlk, qt, blocks, O, K)
    with np.errstate(invalid="ignore", over="ignore"):
        want = x.astype(np.float64) @ wd.astype(np.float64).T
    for got in (run_planar(mlk, qt, x, planar, O),
                np.concatenate([run_planar(mlk, qt, x[t], planar, O) for t in range(T)])):
        for t in (1, 2):
            np.testing.assert_array_equal(np.isnan(got[t]), np.isnan(want[t]))
            fin = np.isfinite(want[t])
            np.testing.assert_array_equal(got[t][~fin & ~np.isnan(want[t])],
                                          want[t][~fin & ~np.isnan(want[t])])
        ok = [0, 3]
        ex, s = dot_exact(x[ok], wd)
        assert_dot_close(got[ok], ex, s, K, f"{qt} finite rows")


@pytest.mark.parametrize("qt", QT)
def test_planar_one_row_equals_block_layout_bound(mlk, orc, qt):
    """One row at the 8B shapes (q/k/v, wo, gate and down): the planar GEMV
    and the block-layout streaming GEMV on the same blocks, both within the
    bound of the exact sums; the planar one needs no workspace."""
    rng = np.random.default_rng(23)
    for O, K in ((6144, 4096), (4096, 4096), (14336, 4096), (4096, 14336)):
        assert mlk.linear_planar_workspace_bytes(1, K, O) == 0
        blocks = orc.quantize(qt, normal(rng, (O, K), 0.02))
        x = normal(rng, (1, K))
        ex, s = dot_exact(x, orc.dequantize(qt, blocks, O, K))
        got_p = run_planar(mlk, qt, x, to_planar(mlk, qt, blocks, O, K), O, workspace=None)
        d_x, d_w = mlk.DeviceBuffer.from_array(x), mlk.DeviceBuffer.from_array(blocks)
        d_y = mlk.DeviceBuffer.empty((1, O))
        mlk.linear_quant(qt, d_x, d_w, d_y, 1, K, O)
        assert_dot_close(got_p, ex, s, K, f"{qt} {O}x{K} planar")
        assert_dot_close(d_y.download(), ex, s, K, f"{qt} {O}x{K} blocks")


STREAM_SHAPES = [  # (out, in, rows, chunk): one call over `out` rows takes more workgroups
    # than the one-shot kernel spreads well (the 8B gate and up as one matrix,
    # 16 tokens, a ragged 5, two token tiles with 24), or one K range with
    # direct output (131088 rows, no split-K partials); `chunk` rows per call
    # stay within the one-shot kernel
    (28672, 4096, 16, 7168), (28672, 4096, 5, 7168), (28672, 4096, 24, 7168),
    (131088, 512, 5, 16384)]


@pytest.mark.parametrize("qt", QT)
@pytest.mark.parametrize("shape", STREAM_SHAPES, ids=["gateup_16", "gateup_5", "gateup_24",
                                                      "direct_5"])
def test_planar_stream_equals_one_shot(mlk, orc, qt, shape):
    """Many row tiles per K range: the streaming launch (each workgroup's
    waves walk the row tiles of one K range, the next tiles' loads in
    flight) forms the same products in the same order as the one-shot
    launch (one workgroup per row group and K range), so one call over all
    rows equals calls over row chunks bit for bit.  The whole result is
    also held to the bound of the exact sums, on a sample of rows."""
    O, K, T, chunk = shape
    rng = np.random.default_rng(O + K + T)
    w = normal(rng, (O, K), 0.02)
    x = normal(rng, (T, K))
    blocks = orc.quantize(qt, w)
    got = run_planar(mlk, qt, x, to_planar(mlk, qt, blocks, O, K), O)
    per_row = blocks.size // O
    parts = []
    for r0 in range(0, O, chunk):
        n = min(chunk, O - r0)
        sub = blocks.reshape(O, per_row)[r0:r0 + n]
        parts.append(run_planar(mlk, qt, x, to_planar(mlk, qt, sub, n, K), n))
    np.testing.assert_array_equal(got, np.concatenate(parts, axis=1))
    rows = np.unique(np.r_[0:64, O // 2 - 32:O // 2 + 32, O - 64:O,
                           rng.choice(O, 256, replace=False)])
    ex, s = dot_exact(x, orc.dequantize(qt, blocks.reshape(O, per_row)[rows], len(rows), K))
    assert_dot_close(got[:, rows], ex, s, K, f"{qt} {shape}")


def test_planar_rejects(mlk, orc):
    """Q4_1 and in_features that are not a multiple of 256 have no planar
    layout; the few-row path needs its workspace."""
    assert mlk.quant_planar_bytes("q4_1", 64, 256) == 0
    assert mlk.quant_planar_bytes("q8_0", 64, 288) == 0
    rng = np.random.default_rng(5)
    blocks = orc.quantize("q8_0", normal(rng, (64, 288), 0.02))
    d_b = mlk.DeviceBuffer.from_array(blocks)
    d_p = mlk.DeviceBuffer(1 << 16, np.uint8)
    with pytest.raises(mlk.MlkError, match="no planar layout"):
        mlk.quant_to_planar("q8_0", d_b, 64, 288, d_p)
    blocks = orc.quantize("q8_0", normal(rng, (64, 512), 0.02))
    planar = to_planar(mlk, "q8_0", blocks, 64, 512)
    need = mlk.linear_planar_workspace_bytes(8, 512, 64)
    small = mlk.DeviceBuffer(need - 256, np.uint8)
    with pytest.raises(mlk.MlkError, match="workspace of"):
        run_planar(mlk, "q8_0", normal(rng, (8, 512)), planar, 64, workspace=small)
