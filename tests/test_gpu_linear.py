"""GPU parity of the linear layers: quantized (Q8_0 / Q4_0 / Q4_1) and F32
linear, and Matmul, through the C ABI.

The bar (written in conftest.assert_dot_close): every output within
gamma_K * sum_k |x_k w_k| of the float64 value of the same product with the
dequantized weights -- the bound any fp32 summation order meets, the
reference's serial loop included.  On the reference's own test inputs the
reference's own tolerance 2e-5 * max(1, |y|) (test/cuda_quant_test.cc:60-66)
is checked as well, and the compiled reference's outputs (tests/golden)
are held to the same bound.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_dot_close, dot_exact, golden

pytestmark = pytest.mark.gpu

QT = ("q8_0", "q4_0", "q4_1")


def normal(rng, shape, std=1.0):
    return (rng.standard_normal(shape) * std).astype(np.float32)


def run_quant(mlk, qt, x, blocks, out_f, bias=None, workspace="auto"):
    x = np.atleast_2d(np.ascontiguousarray(x, np.float32))
    T, K = x.shape
    d_x = mlk.DeviceBuffer.from_array(x)
    d_w = mlk.DeviceBuffer.from_array(np.ascontiguousarray(blocks, np.uint8))
    d_b = None if bias is None else mlk.DeviceBuffer.from_array(np.asarray(bias, np.float32))
    d_y = mlk.DeviceBuffer.empty((T, out_f))
    mlk.linear_quant(qt, d_x, d_w, d_y, T, K, out_f, bias=d_b, workspace=workspace)
    return d_y.download()


def near_reference_tolerance(got, exact):
    """test/cuda_quant_test.cc:60-66."""
    got = np.atleast_2d(np.asarray(got, np.float64))
    assert (np.abs(got - exact) <= 2e-5 * np.maximum(1.0, np.abs(exact))).all()


def test_quant_linear_reference_patterns(mlk, orc):
    """The weight / input patterns and shapes of the reference's own tests
    (131 outputs, in 1, 17, 32, 33, 65; one and three rows; bias), against
    float64 and the compiled reference's outputs."""
    g = golden("linear")
    for qt in QT:
        for inf in (1, 17, 32, 33, 65):
            blocks = g[f"p43_{qt}_{inf}_w"]
            w = orc.dequantize(qt, blocks, 131, inf)
            for rows in (1, 3):
                x = g[f"p43_{qt}_{inf}_x{rows}"]
                ex, s = dot_exact(x, w)
                got = run_quant(mlk, qt, x, blocks, 131)
                assert_dot_close(got, ex, s, inf, f"{qt} in={inf} rows={rows}")
                near_reference_tolerance(got, ex)
                assert_dot_close(g[f"p43_{qt}_{inf}_y{rows}"], ex, s, inf, "reference itself")
                bias = np.linspace(-1, 1, 131).astype(np.float32)
                got = run_quant(mlk, qt, x, blocks, 131, bias=bias)
                exb, sb = dot_exact(x, w, bias)
                assert_dot_close(got, exb, sb, inf + 1, f"{qt} in={inf} bias")
        for cols in (32, 86):
            blocks, x = g[f"sin_{qt}_{cols}_w"], g[f"sin_{qt}_{cols}_x"]
            ex, s = dot_exact(x, orc.dequantize(qt, blocks, 7, cols))
            assert_dot_close(run_quant(mlk, qt, x, blocks, 7), ex, s, cols, f"{qt} sin {cols}")


@pytest.mark.parametrize("qt", QT)
@pytest.mark.parametrize("shape", [(131, 64, 1), (4099, 4096, 1), (64, 4096, 2), (37, 4096, 3),
                                   (16, 4096, 4), (33, 14336, 5), (200, 128, 9), (5, 96, 2),
                                   (1, 4096, 1), (4096, 320, 2), (4095, 4096, 1), (8193, 1056, 3),
                                   (1024, 4096, 4), (4096, 4096, 7)])
def test_quant_linear_shapes(mlk, orc, qt, shape):
    """The split-K path: whole and partial last spans (in % 256 and % 512 !=
    0, masked per lane), partial last workgroups of 2 and 4 rows (out odd,
    out around 4096 where the rows per workgroup change), token counts 1..7
    (launches of up to 4 rows); 9 rows take the GEMM."""
    O, K, T = shape
    rng = np.random.default_rng(O * 7 + K + T)
    w = normal(rng, (O, K), 0.02)
    blocks = orc.quantize(qt, w)
    x = normal(rng, (T, K))
    bias = normal(rng, (O,), 0.1)
    ex, s = dot_exact(x, orc.dequantize(qt, blocks, O, K), bias)
    got = run_quant(mlk, qt, x, blocks, O, bias=bias)
    assert_dot_close(got, ex, s, K + 1, f"{qt} {shape}")
    # the compiled reference's (oracle's) own result meets the same bound
    assert_dot_close(orc.linear_quant(qt, x, blocks, O, bias=bias), ex, s, K + 1, "oracle")


STREAM_SHAPES = [  # (out, in): one token row, in % 64 == 0 and x within 64 KiB of LDS
    (14336, 4096), (4096, 14336), (8193, 8192), (5, 4160), (3, 64), (14337, 128),
    (4096, 15360), (1, 4096), (300, 16384)]


@pytest.mark.parametrize("qt", QT)
@pytest.mark.parametrize("shape", STREAM_SHAPES)
def test_quant_linear_decode_row(mlk, orc, qt, shape):
    """One token row takes the streaming GEMV (two-block pieces per lane, x
    in LDS, the next step's loads ahead of the current one): whole 4096-input
    passes and a partial last pass (in 4160, 14336: lanes past the row's last
    piece masked), several row groups per wave (out 14337 over in 128), odd
    out with two rows per wave, and in 16384, whose x does not fit the LDS,
    on the split-K kernel."""
    O, K = shape
    rng = np.random.default_rng(O + 3 * K)
    w = normal(rng, (O, K), 0.02)
    blocks = orc.quantize(qt, w)
    x = normal(rng, (1, K))
    bias = normal(rng, (O,), 0.1)
    ex, s = dot_exact(x, orc.dequantize(qt, blocks, O, K), bias)
    got = run_quant(mlk, qt, x, blocks, O, bias=bias)
    assert_dot_close(got, ex, s, K + 1, f"{qt} {shape}")
    got2 = run_quant(mlk, qt, x, blocks, O)
    ex2, s2 = dot_exact(x, orc.dequantize(qt, blocks, O, K))
    assert_dot_close(got2, ex2, s2, K, f"{qt} {shape} no bias")


GEMM_SHAPES = [  # (out, in, rows): 8 rows and more take the matrix-core GEMM
    (4096, 4096, 128), (1024, 4096, 200), (131, 64, 32), (4097, 96, 33), (300, 4128, 257),
    (14336, 4096, 64), (4096, 14336, 96), (4096, 4096, 1024)]


@pytest.mark.parametrize("wt", QT + ("f32",))
@pytest.mark.parametrize("shape", GEMM_SHAPES)
def test_linear_gemm_shapes(mlk, orc, wt, shape):
    """The GEMM path: whole and partial 128-row / 128-output tiles (rows 32,
    33, 200, 257; outputs 131, 300, 4097), one to 448 K stages of 32 (in
    4128 = 129 stages: an odd count, so the last stage reads the second LDS
    buffer), the layer's projection shapes, bias.  Each shape runs with the
    split-K workspace (when the shape uses one: splits of whole stages, the
    last one shorter at in = 4128) and without it."""
    O, K, T = shape
    rng = np.random.default_rng(O * 3 + K + T)
    w = normal(rng, (O, K), 0.02)
    x = normal(rng, (T, K))
    bias = normal(rng, (O,), 0.1)
    ws_bytes = mlk.linear_workspace_bytes(T, K, O)
    outs = []
    for workspace in ("auto", None):
        if wt == "f32":
            ex, s = dot_exact(x, w, bias)
            got = run_f32(mlk, x, w, bias, workspace=workspace)
        else:
            blocks = orc.quantize(wt, w)
            ex, s = dot_exact(x, orc.dequantize(wt, blocks, O, K), bias)
            got = run_quant(mlk, wt, x, blocks, O, bias=bias, workspace=workspace)
        assert_dot_close(got, ex, s, K + 1, f"{wt} {shape} workspace={workspace}")
        rel = np.abs(got - ex) / s
        print(f"gemm {wt} {shape} workspace={workspace} ({ws_bytes} B): "
              f"max |err| / sum|terms| = {float(rel.max()):.2e}")
        outs.append(got)
    if ws_bytes == 0:  # no split: the same kernel, the same order
        np.testing.assert_array_equal(outs[0], outs[1])


@pytest.mark.parametrize("wt", ("q8_0", "q4_0"))
def test_linear_gemm_wide_tiles(mlk, orc, wt):
    """Q8_0 / Q4_0 tiles on bf16 piece products with 256 outputs per
    workgroup: 4059 rows x 4300 outputs is 32 x 17 = 544 such tiles, at least
    two per compute unit on the 256 of an MI355X, so the launch takes them
    (no split of K = 256). The last row tile and the last output tile are
    partial. Same bar as the other GEMM shapes, with a bias."""
    O, K, T = 4300, 256, 4059
    rng = np.random.default_rng(41)
    w = normal(rng, (O, K), 0.02)
    x = normal(rng, (T, K))
    bias = normal(rng, (O,), 0.1)
    blocks = orc.quantize(wt, w)
    ex, s = dot_exact(x, orc.dequantize(wt, blocks, O, K), bias)
    got = run_quant(mlk, wt, x, blocks, O, bias=bias)
    assert_dot_close(got, ex, s, K + 1, f"{wt} wide tiles")


BENCH_GEMM_SHAPES = [(4096, 14336, 4096), (14336, 4096, 4096)]  # (out, in, rows)


def sample_rows(T, tile=128):
    """Rows spread over every 128-row tile: its first, a middle and its last
    row (the last tile's rows may be fewer)."""
    rows = set()
    for r0 in range(0, T, tile):
        r1 = min(T, r0 + tile) - 1
        rows.update((r0, (r0 + r1) // 2 + 1 if r1 > r0 else r0, r1))
    return np.array(sorted(rows))


@pytest.mark.parametrize("wt", ("q8_0", "q4_0"))
@pytest.mark.parametrize("shape", BENCH_GEMM_SHAPES, ids=["down_4096x14336", "gate_14336x4096"])
def test_linear_gemm_bench_shapes(mlk, orc, wt, shape):
    """The prefill layer's GEMM at the shapes the bench times (T = 4096
    tokens; w_down: 4096 outputs over 14336 inputs, w_gate / w_up: 14336
    outputs over 4096): 32 row tiles x 16 or 56 output tiles of 256 is at
    least two workgroups per compute unit, so these take the 8-wave
    piece-product tiles.  Every output of 96 rows (first, middle and last of
    each of the 32 row tiles) against the gamma_K bound of the float64
    products with the dequantized weights."""
    O, K, T = shape
    rng = np.random.default_rng(O + 2 * K)
    w = normal(rng, (O, K), 0.02)
    blocks = orc.quantize(wt, w)
    del w
    x = normal(rng, (T, K))
    got = run_quant(mlk, wt, x, blocks, O)
    rows = sample_rows(T)
    assert rows.size >= 64
    ex, s = dot_exact(x[rows], orc.dequantize(wt, blocks, O, K))
    assert_dot_close(got[rows], ex, s, K, f"{wt} {shape} sampled rows")
    assert np.isfinite(got).all()
    print(f"gemm {wt} {shape}: {rows.size} rows x {O} outputs checked; "
          f"max |err| / sum|terms| = {float((np.abs(got[rows] - ex) / s).max()):.2e}")


@pytest.mark.parametrize("wt", ("q8_0", "q4_0"))
@pytest.mark.parametrize("shape", [(300, 512, 130), (4300, 256, 4059)],
                         ids=["128_output_tiles", "256_output_tiles"])
def test_linear_gemm_non_finite_inputs(mlk, orc, wt, shape):
    """The piece-product GEMM (Q8_0 / Q4_0, more than 64 rows, in a multiple
    of 256) with inf and NaN in x: row 0, a middle row and a row of the
    partial last row tile.  Every output those rows reach is what the
    products give (the same NaN pattern, infinities of the same sign); every
    other row stays finite and within the bound.  Both tile widths: 300
    outputs over 130 rows (128-output tiles), and 4300 outputs over 4059
    rows (enough tiles for the 256-output ones)."""
    O, K, T = shape
    rng = np.random.default_rng(O + K + T)
    blocks = orc.quantize(wt, normal(rng, (O, K), 0.02))
    wd = orc.dequantize(wt, blocks, O, K)
    x = normal(rng, (T, K))
    bad_rows = [0, T // 2, T - 1]
    x[0, 7] = np.nan
    x[T // 2, 3] = -np.inf
    x[T - 1, K - 1] = np.inf
    got = run_quant(mlk, wt, x, blocks, O)
    with np.errstate(invalid="ignore", over="ignore"):
        want = x[bad_rows].astype(np.float64) @ wd.astype(np.float64).T
    for i, t in enumerate(bad_rows):
        np.testing.assert_array_equal(np.isnan(got[t]), np.isnan(want[i]), err_msg=f"row {t}")
        inf = np.isinf(want[i])
        np.testing.assert_array_equal(got[t][inf], want[i][inf], err_msg=f"row {t}")
    ok = np.setdiff1d(sample_rows(T), bad_rows)
    ex, s = dot_exact(x[ok], wd)
    assert_dot_close(got[ok], ex, s, K, f"{wt} {shape} finite rows")


SKINNY_SHAPES = [  # (out, in, rows): quantized weights with 8..32 rows, in a multiple of 256, take
    # the skinny kernel (F32 runs the tiled GEMM on the same shapes)
    (4096, 4096, 8), (1024, 4096, 9), (100, 256, 16), (4097, 512, 17), (64, 4096, 31),
    (14336, 4096, 32), (4096, 14336, 12), (130, 768, 25)]


@pytest.mark.parametrize("wt", QT + ("f32",))
@pytest.mark.parametrize("shape", SKINNY_SHAPES)
def test_linear_skinny_shapes(mlk, orc, wt, shape):
    """The skinny path (W streamed straight into MFMA registers): 16- and
    32-row token tiles (rows 8..32, partial tiles), output counts not a
    multiple of the 64-row workgroup (100, 130, 4097), one to 56 K chunks,
    split-K over the workspace and unsplit."""
    O, K, T = shape
    rng = np.random.default_rng(O + 5 * K + T)
    w = normal(rng, (O, K), 0.02)
    x = normal(rng, (T, K))
    bias = normal(rng, (O,), 0.1)
    if wt == "f32":
        ex, s = dot_exact(x, w, bias)
    else:
        blocks = orc.quantize(wt, w)
        ex, s = dot_exact(x, orc.dequantize(wt, blocks, O, K), bias)
    for workspace in ("auto", None):
        got = (run_f32(mlk, x, w, bias, workspace=workspace) if wt == "f32" else
               run_quant(mlk, wt, x, blocks, O, bias=bias, workspace=workspace))
        assert_dot_close(got, ex, s, K + 1, f"{wt} {shape} workspace={workspace}")


def test_linear_workspace_sizes(mlk):
    """The split-K workspace: none below 8 rows (GEMV) or when the tiles
    already fill the GPU, splits * rows * out * 4 bytes otherwise; a
    workspace smaller than asked for is ignored (no split), not overrun."""
    assert mlk.linear_workspace_bytes(7, 4096, 4096) == 0
    assert mlk.linear_workspace_bytes(8, 4096, 4096) > 0
    assert mlk.linear_workspace_bytes(4096, 4096, 4096) == 0  # 1024 tiles
    b = mlk.linear_workspace_bytes(128, 4096, 4096)
    assert b > 0 and b % (128 * 4096 * 4) == 0
    rng = np.random.default_rng(9)
    O, K, T = 1024, 4096, 64
    w = normal(rng, (O, K), 0.02)
    x = normal(rng, (T, K))
    ex, s = dot_exact(x, w)
    need = mlk.linear_workspace_bytes(T, K, O)
    small = mlk.DeviceBuffer(need - 16, np.uint8)
    exact = mlk.DeviceBuffer(need, np.uint8)
    assert_dot_close(run_f32(mlk, x, w, workspace=small), ex, s, K, "workspace too small")
    assert_dot_close(run_f32(mlk, x, w, workspace=exact), ex, s, K, "workspace of the size")


def test_linear_gemm_f32_ragged_in(mlk):
    """fp32 weights with in_features % 32 != 0 (the last stage is partly
    masked) on the GEMM path."""
    rng = np.random.default_rng(8)
    for O, K, T in ((200, 100, 40), (129, 36, 130), (64, 4100, 64)):
        w = normal(rng, (O, K), 0.02)
        x = normal(rng, (T, K))
        ex, s = dot_exact(x, w)
        assert_dot_close(run_f32(mlk, x, w), ex, s, K, f"f32 ragged {O}x{K} T={T}")


@pytest.mark.parametrize("qt", QT)
@pytest.mark.parametrize("T", [1, 2])
def test_quant_linear_special_scales(mlk, orc, qt, T):
    """Subnormal, zero and large fp16 scales (and Q4_1 minima) decode like the
    CPU, on the streaming (one row) and split-K kernels: blocks are
    hand-made, then checked against float64."""
    rng = np.random.default_rng(1)
    O, K = 8, 256
    blocks = orc.quantize(qt, normal(rng, (O, K), 0.02)).reshape(O, K // 32, -1).copy()
    scales = [0x0001, 0x03FF, 0x0000, 0x7BFF, 0x3C00, 0x8001, 0x0400, 0x1234]
    for j in range(O):
        blocks[j, :, 0:2] = np.array([scales[j]], np.uint16).view(np.uint8)
        if qt == "q4_1":
            blocks[j, :, 2:4] = np.array([scales[(j + 3) % O]], np.uint16).view(np.uint8)
    blocks = blocks.reshape(-1)
    x = normal(rng, (T, K), 1e-3)
    ex, s = dot_exact(x, orc.dequantize(qt, blocks, O, K))
    assert_dot_close(run_quant(mlk, qt, x, blocks, O), ex, s, K, f"{qt} scales")


def test_quant_linear_unaligned_buffers(mlk, orc):
    """x not 16-byte aligned and blocks only 2-byte aligned take the
    byte-load path and give the same result."""
    rng = np.random.default_rng(2)
    O, K, T = 19, 128, 3
    for qt in QT:
        blocks = orc.quantize(qt, normal(rng, (O, K), 0.02))
        x = normal(rng, (T, K))
        ex, s = dot_exact(x, orc.dequantize(qt, blocks, O, K))
        xb = mlk.DeviceBuffer(x.nbytes + 4, np.uint8)
        wb = mlk.DeviceBuffer(blocks.nbytes + 2, np.uint8)
        mlk.check(mlk.lib.mlk_memcpy(xb.ptr + 4, x.ctypes.data, x.nbytes, mlk.H2D))
        mlk.check(mlk.lib.mlk_memcpy(wb.ptr + 2, blocks.ctypes.data, blocks.nbytes, mlk.H2D))
        y = mlk.DeviceBuffer.empty((T, O))
        mlk.linear_quant(qt, xb.ptr + 4, wb.ptr + 2, y, T, K, O)
        assert_dot_close(y.download(), ex, s, K, f"{qt} unaligned")


def test_quant_linear_chains_device_outputs(mlk, orc):
    """test/cuda_quant_test.cc:130-148: the device output of one linear is the
    next one's input."""
    rng = np.random.default_rng(4)
    for qt in QT:
        w1, w2 = normal(rng, (128, 192), 0.05), normal(rng, (7, 128), 0.05)
        b1, b2 = orc.quantize(qt, w1), orc.quantize(qt, w2)
        x = normal(rng, (3, 192))
        d_x = mlk.DeviceBuffer.from_array(x)
        d_h = mlk.DeviceBuffer.empty((3, 128))
        d_y = mlk.DeviceBuffer.empty((3, 7))
        mlk.linear_quant(qt, d_x, mlk.DeviceBuffer.from_array(b1), d_h, 3, 192, 128)
        mlk.linear_quant(qt, d_h, mlk.DeviceBuffer.from_array(b2), d_y, 3, 128, 7)
        h = d_h.download()
        ex, s = dot_exact(h, orc.dequantize(qt, b2, 7, 128))
        assert_dot_close(d_y.download(), ex, s, 128, f"{qt} second layer")


def run_f32(mlk, x, w, bias=None, workspace="auto"):
    x = np.atleast_2d(x)
    d_y = mlk.DeviceBuffer.empty((x.shape[0], w.shape[0]))
    d_b = None if bias is None else mlk.DeviceBuffer.from_array(bias)
    mlk.linear_f32(mlk.DeviceBuffer.from_array(x), mlk.DeviceBuffer.from_array(w), d_y,
                   x.shape[0], x.shape[1], w.shape[0], bias=d_b, workspace=workspace)
    return d_y.download()


def test_f32_linear_and_matmul(mlk, orc):
    g = golden("linear")
    x, w, b = g["f32_x"], g["f32_w"], g["f32_bias"]
    ex, s = dot_exact(x, w)
    assert_dot_close(run_f32(mlk, x, w), ex, s, 33, "tests/test_cuda_linear.cc shape")
    ex, s = dot_exact(x, w, b)
    assert_dot_close(run_f32(mlk, x, w, b), ex, s, 34, "bias")
    rng = np.random.default_rng(6)
    for O, K, T in ((4096, 4096, 1), (1000, 4096, 3), (77, 1000, 6), (9, 35, 2), (3, 14336, 4),
                    (4097, 100, 3), (14336, 4096, 2), (5, 260, 5)):
        w = normal(rng, (O, K), 0.02)
        x = normal(rng, (T, K))
        bias = normal(rng, (O,))
        ex, s = dot_exact(x, w, bias)
        assert_dot_close(run_f32(mlk, x, w, bias), ex, s, K + 1, f"f32 {O}x{K} T={T}")
    for m, k, n in ((3, 7, 5), (1, 33, 17)):
        a, bm = g[f"mm_{m}x{k}x{n}_a"], g[f"mm_{m}x{k}x{n}_b"]
        c = mlk.DeviceBuffer.empty((m, n))
        mlk.matmul(mlk.DeviceBuffer.from_array(a), mlk.DeviceBuffer.from_array(bm), c, m, k, n)
        ex, s = dot_exact(a, bm.T)
        assert_dot_close(c.download(), ex, s, k, "matmul")
    a, bm = normal(rng, (70, 300)), normal(rng, (300, 45))
    c = mlk.DeviceBuffer.empty((70, 45))
    mlk.matmul(mlk.DeviceBuffer.from_array(a), mlk.DeviceBuffer.from_array(bm), c, 70, 300, 45)
    ex, s = dot_exact(a, bm.T)
    assert_dot_close(c.download(), ex, s, 300, "matmul 70x300x45")
