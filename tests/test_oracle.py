"""Pins the CPU oracle before it is trusted as the checker.

Each oracle function is checked against something that does not restate it:
  - the reference's own golden vectors (tests/golden, written by the
    reference sources compiled in place);
  - the reference's known-answer tests (values copied as data from
    test/ops_test.cc, test/quantized_tensor_test.cc, test/test_quant.cc);
  - mathematics: IEEE binary16 via numpy, float64 closed forms, rotation
    invariants (identity at pos 0, composition, norm preservation);
  - the compiled reference itself on random inputs (when oracle/_ref is
    built, i.e. in the container that has the reference tree).
The planted-mistake tests at the end show the checks are sharp enough: a
dropped term, a flipped sign or a swapped index in a copy of an oracle
formula fails them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle as O
from conftest import assert_bits_equal, golden

QT = ("q8_0", "q4_0", "q4_1")


def near(actual, expected, tol=2e-5):
    """test/ops_test.cc:44-47: |a - e| <= 2e-5 * max(1, |e|)."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert np.isfinite(actual).all()
    assert (np.abs(actual - expected) <= tol * np.maximum(1.0, np.abs(expected))).all(), \
        (actual, expected)


# ------------------------------------------------------------------- fp16

def test_fp16_decode_exhaustive_against_ieee(orc):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.fp16_to_fp32_array(codes)
    want = codes.view(np.float16).astype(np.float32)
    finite = ~np.isnan(want)
    assert_bits_equal(got[finite], want[finite], "fp16 -> fp32")
    # NaN codes keep sign and payload: bits = sign | 0x7F800000 | frac << 13
    nan_codes = codes[~finite].astype(np.uint32)
    expect_bits = ((nan_codes & 0x8000) << 16) | 0x7F800000 | ((nan_codes & 0x3FF) << 13)
    np.testing.assert_array_equal(got[~finite].view(np.uint32), expect_bits)


def test_fp16_decode_reference_codes(orc):
    """Codes used by the reference tests (0.5 = 0x3800, -1 = 0xBC00, ...)."""
    for code, value in ((0x3800, 0.5), (0xBC00, -1.0), (0x3C00, 1.0), (0x0001, 2.0 ** -24),
                        (0x3400, 0.25), (0x3A00, 0.75), (0x4000, 2.0), (0xC000, -2.0),
                        (0xB800, -0.5), (0x3E00, 1.5), (0x0000, 0.0), (0x7BFF, 65504.0)):
        assert orc.fp16_to_fp32(code) == value


def test_fp16_encode_matches_ieee_round_to_nearest_even(orc):
    """All 8192 rounding remainders for every exponent and sign at mantissa
    heads that exercise carries, plus 2^24 random patterns; numpy's float16
    cast is IEEE round-to-nearest-even with overflow to inf."""
    heads = np.array([0, 1, 2, 0x1FF, 0x200, 0x3FE, 0x3FF], np.uint32)
    rem = np.arange(8192, dtype=np.uint32)
    exps = np.arange(255, dtype=np.uint32)  # finite exponents
    man = (heads[:, None] << 13 | rem[None, :]).reshape(-1)
    bits = (exps[:, None] << 23 | man[None, :]).reshape(-1)
    bits = np.concatenate([bits, bits | 0x80000000])
    rng = np.random.default_rng(0)
    rand = rng.integers(0, 2 ** 32, size=1 << 24, dtype=np.uint64).astype(np.uint32)
    rand = rand[((rand >> 23) & 255) != 255]
    for b in (bits, rand):
        x = b.view(np.float32)
        got = orc.fp32_to_fp16_array(x)
        with np.errstate(over="ignore"):
            want = x.astype(np.float16).view(np.uint16)
        np.testing.assert_array_equal(got, want)


def test_fp16_encode_specials(orc):
    f = np.array([np.inf, -np.inf, 65504.0, 65520.0, -65520.0, 2.0 ** -25,
                  2.0 ** -25 * 1.0000001, 2.0 ** -24, 1e-30, -0.0], np.float32)
    got = orc.fp32_to_fp16_array(f)
    np.testing.assert_array_equal(
        got, [0x7C00, 0xFC00, 0x7BFF, 0x7C00, 0xFC00, 0x0000, 0x0001, 0x0001, 0x0000, 0x8000])
    # NaN: quiet, sign and top payload kept
    nan = np.array([0x7F800001, 0xFFC00000, 0x7FFFFFFF], np.uint32).view(np.float32)
    h = orc.fp32_to_fp16_array(nan).astype(np.uint32)
    assert ((h & 0x7C00) == 0x7C00).all() and ((h & 0x0200) != 0).all()
    assert list(h >> 15) == [0, 1, 0]


# --------------------------------------------------------------- quant

@pytest.mark.parametrize("qt", QT)
def test_quantizers_match_reference_golden(orc, qt):
    g = golden("quant")
    for name in ("c4", "ragged100", "ragged33", "ragged7", "edge"):
        x = g[f"{name}_x"]
        np.testing.assert_array_equal(orc.quantize(qt, x), g[f"{name}_{qt}_blocks"], name)
        deq = orc.dequantize(qt, g[f"{name}_{qt}_blocks"], *x.shape)
        assert_bits_equal(deq, g[f"{name}_{qt}_deq"], f"{name} dequant")


@pytest.mark.parametrize("qt", QT)
def test_dequant_golden_handcrafted_blocks(orc, qt):
    g = golden("dequant_kat")
    rows, cols = int(g["rows"]), int(g["cols"])
    deq = orc.dequantize(qt, g[f"{qt}_blocks"], rows, cols)
    assert_bits_equal(deq, g[f"{qt}_deq"], "row-wise overload")
    assert_bits_equal(deq, g[f"{qt}_deq_flat"], "QuanTensor overload")


@pytest.mark.parametrize("qt", QT)
def test_dequant_closed_form_float64(orc, qt):
    """test/test_quant.cc:388-417 ReferenceFp16 / ReferenceQuantWeight, in
    float64 with ldexp, over random blocks with every scale class."""
    bb = O.BLOCK_BYTES[qt]
    rng = np.random.default_rng(3)
    nb = 400
    raw = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    scales = rng.integers(0, 0x7C00, size=nb).astype(np.uint16)  # finite codes incl. subnormal
    raw[:, 0] = scales & 0xFF
    raw[:, 1] = scales >> 8
    if qt == "q4_1":
        mins = rng.integers(0, 0x7C00, size=nb).astype(np.uint16) | (rng.integers(0, 2, nb) << 15)
        raw[:, 2] = mins & 0xFF
        raw[:, 3] = mins >> 8

    def ref16(code):
        e, f = (code >> 10) & 31, code & 1023
        v = math.ldexp(f, -24) if e == 0 else math.ldexp(1024 + f, e - 25)
        return -v if code & 0x8000 else v

    got = orc.dequantize(qt, raw.reshape(-1), nb, 32)
    for b in range(nb):
        d = ref16(int(raw[b, 0]) | int(raw[b, 1]) << 8)
        for i in range(32):
            if qt == "q8_0":
                want = d * int(np.int8(raw[b, 2 + i]))
            else:
                base = 2 if qt == "q4_0" else 4
                byte = int(raw[b, base + (i & 15)])
                code = (byte & 15) if i < 16 else (byte >> 4)
                want = d * (code - 8) if qt == "q4_0" else \
                    d * code + ref16(int(raw[b, 2]) | int(raw[b, 3]) << 8)
            # exact for Q8_0/Q4_0; Q4_1 rounds d*code + m once to float
            assert got[b, i] == np.float32(want), (b, i, got[b, i], want)


def test_dequant_reference_kats(orc):
    """test/quantized_tensor_test.cc:179-303."""
    q8 = np.zeros(34, np.uint8)
    q8[0:2] = [0x00, 0x38]                       # d = 0.5
    q8[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    np.testing.assert_array_equal(orc.dequantize("q8_0", q8, 1, 32)[0], 0.5 * (np.arange(32) - 16))
    q40 = np.zeros(18, np.uint8)
    q40[0:2] = [0x00, 0x38]
    i = np.arange(16)
    q40[2:] = ((15 - i) << 4) | i
    y = orc.dequantize("q4_0", q40, 1, 32)[0]
    np.testing.assert_array_equal(y[:16], 0.5 * (i - 8))
    np.testing.assert_array_equal(y[16:], 0.5 * (7 - i))
    q41 = np.zeros(20, np.uint8)
    q41[0:4] = [0x00, 0x38, 0x00, 0xBC]          # d = 0.5, m = -1
    q41[4:] = (i << 4) | i
    y = orc.dequantize("q4_1", q41, 1, 32)[0]
    np.testing.assert_array_equal(y[:16], 0.5 * i - 1)
    np.testing.assert_array_equal(y[16:], 0.5 * i - 1)


def test_quantizer_reference_invariants(orc):
    """test/test_quant.cc: zero blocks, tail padding, round trips."""
    z = orc.quantize("q8_0", np.zeros(64, np.float32)).reshape(2, 34)
    assert (z == 0).all()
    q40 = orc.quantize("q4_0", np.full(100, 0.5, np.float32)).reshape(4, 18)
    last = q40[-1, 2:]
    assert ((last >> 4) == 8).all() and ((last[4:] & 15) == 8).all()
    q41 = orc.quantize("q4_1", np.full(100, 0.5, np.float32)).reshape(4, 20)
    assert q41[-1, 2] == 0 and q41[-1, 3] == 0         # tail min is the zero padding
    assert (q41[-1, 0] | q41[-1, 1]) != 0
    q80 = orc.quantize("q8_0", np.full(100, 0.5, np.float32)).reshape(4, 34)
    assert (q80[-1, 2 + 4:] == 0).all()
    src = ((np.arange(64) % 19 - 9) * 0.3).astype(np.float32)
    src[0], src[32] = -4.0, 4.0
    back = orc.dequantize("q8_0", orc.quantize("q8_0", src.reshape(2, 32)), 2, 32)
    assert np.abs(back.reshape(-1) - src).max() <= 0.02
    for qt, tol in (("q8_0", 0.01), ("q4_0", 0.1), ("q4_1", 0.05)):
        for shape in ((1, 100), (32, 86), (2, 35), (2, 48), (2, 49)):
            rows, cols = shape
            r = np.arange(rows)[:, None]
            c = np.arange(cols)[None, :]
            v = (0.8 + r * 0.005 + 0.2 * np.sin(c * 0.17) + 0.1 * np.cos(c * 0.11)).astype(np.float32)
            v = np.where(r % 2 == 0, v, -v).astype(np.float32)
            back = orc.dequantize(qt, orc.quantize(qt, v), rows, cols)
            assert np.abs(back - v).max() <= tol, (qt, shape)


def test_gather_is_row_copy_and_rejects_bad_ids(orc):
    rng = np.random.default_rng(1)
    t = rng.standard_normal((131, 64)).astype(np.float32)
    ids = np.array([0, 1, 130, 128, 5], np.int32)
    assert_bits_equal(orc.gather_f32(t, ids), t[ids], "gather")
    for bad in ([131], [-1]):
        with pytest.raises(ValueError):
            orc.gather_f32(t, np.array(bad, np.int32))
    blocks = orc.quantize("q4_1", t)
    assert_bits_equal(orc.gather_quant("q4_1", blocks, 131, 64, ids),
                      orc.dequantize("q4_1", blocks, 131, 64)[ids], "quant gather")


# -------------------------------------------------------------- rmsnorm

def rms_closed_form(x, w, eps):
    x = np.asarray(x, np.float64)
    den = math.sqrt(float(np.sum(x * x)) / x.size + eps)
    return x / den * np.asarray(w, np.float64)


def test_rmsnorm_reference_kats(orc):
    """test/ops_test.cc:158-188."""
    near(orc.rmsnorm(np.array([3, 4], np.float32), np.ones(2, np.float32), 0.0),
         [0.8485281374, 1.1313708499])
    v, w = [-2, 0.25, 3.5], [0.5, 2, -1]
    near(orc.rmsnorm(np.array(v, np.float32), np.array(w, np.float32), 1e-5),
         rms_closed_form(v, w, 1e-5))
    big = np.finfo(np.float32).max
    tiny = np.float32(np.finfo(np.float32).smallest_subnormal)
    for x in ([big, -big], [tiny, 2 * tiny]):
        x = np.array(x, np.float32)
        near(orc.rmsnorm(x, np.ones(2, np.float32), 0.0), rms_closed_form(x, [1, 1], 0.0))
    near(orc.rmsnorm(np.zeros(2, np.float32), np.ones(2, np.float32), 1e-5), [0, 0])
    for eps in (-1.0, float("nan"), float("inf")):
        with pytest.raises(ValueError):
            orc.rmsnorm(np.array([3, 4], np.float32), np.ones(2, np.float32), eps)
    with pytest.raises(ValueError):  # 0 / 0: denominator must be positive
        orc.rmsnorm(np.zeros(2, np.float32), np.ones(2, np.float32), 0.0)


def test_rmsnorm_against_golden_and_closed_form(orc):
    g = golden("rows_8b_70b")
    for tag in ("8b", "70b"):
        x, w, y = g[f"rms_{tag}_x"], g[f"rms_{tag}_w"], g[f"rms_{tag}_y"]
        assert_bits_equal(orc.rmsnorm(x, w, 1e-5), y, f"golden {tag}")
        near(y, rms_closed_form(x, w, 1e-5), tol=1e-6)


def test_add_rmsnorm_is_add_then_norm(orc):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 50)).astype(np.float32)
    d = rng.standard_normal((3, 50)).astype(np.float32)
    w = rng.standard_normal(50).astype(np.float32)
    r, y = orc.add_rmsnorm(x, d, w, 1e-5)
    assert_bits_equal(r, x + d, "residual")
    for i in range(3):
        near(y[i], rms_closed_form(x[i] + d[i], w, 1e-5), tol=1e-6)


# ----------------------------------------------------------------- rope

KAT_NORMAL = ([-1.1426396637476532, 1.922075596544176, 2.585678829246765, 4.279516911052588],
              [-1.501340104140228, -1.4127908166817231, 1.2945044152185103, -2.8851790791872496])
KAT_NEOX = ([-1.9841106485555495, 1.590674663968739, 2.4623779024123156, 4.17968349440576],
            [-1.922075596544176, 0.7970023325794974, -1.1426396637476532, -2.9350957875106634])


@pytest.mark.parametrize("rt,kat", [(O.ROPE_NORMAL, KAT_NORMAL), (O.ROPE_NEOX, KAT_NEOX)])
def test_rope_reference_kats(orc, rt, kat):
    """test/ops_test.cc:749-769: pos 1, theta 100 rotates by 1 and 0.1 rad."""
    q = np.array([[1, 2, 3, 4]], np.float32)
    k = np.array([[-2, 0.5, 1, -3]], np.float32)
    gq, gk = orc.rope(q, k, 1, 1, 4, pos0=1, theta=100.0, rope_type=rt)
    near(gq[0], kat[0])
    near(gk[0], kat[1])


@pytest.mark.parametrize("rt", [O.ROPE_NORMAL, O.ROPE_NEOX])
def test_rope_invariants(orc, rt):
    """test/ops_test.cc:734-833: identity at pos 0, per-head independence,
    composition 3 + 4 = 7, norm preservation."""
    q = np.array([[1, 2, -3, 4, -2, 0.5, 1, -3]], np.float32)
    k = np.array([[3, -2, 1, 0.25]], np.float32)
    gq, gk = orc.rope(q, k, 2, 1, 4, pos0=0, theta=100.0, rope_type=rt)
    assert_bits_equal(gq, q, "pos 0 q")
    assert_bits_equal(gk, k, "pos 0 k")
    q3, k3 = orc.rope(q, k, 2, 1, 4, pos0=3, theta=100.0, rope_type=rt)
    q7a, k7a = orc.rope(q3, k3, 2, 1, 4, pos0=4, theta=100.0, rope_type=rt)
    q7, k7 = orc.rope(q, k, 2, 1, 4, pos0=7, theta=100.0, rope_type=rt)
    near(q7a, q7)
    near(k7a, k7)
    for a, b in ((q.reshape(2, 4), q7.reshape(2, 4)), (k.reshape(1, 4), k7.reshape(1, 4))):
        near((b.astype(np.float64) ** 2).sum(1), (a.astype(np.float64) ** 2).sum(1))
    one, _ = orc.rope(q[:, 4:], np.zeros((1, 4), np.float32), 1, 1, 4, pos0=7, theta=100.0,
                      rope_type=rt)
    near(q7[:, 4:], one)


def test_rope_golden_and_positions(orc):
    g = golden("rows_8b_70b")
    for pos in (0, 1, 4095, 8191):
        q, k = g[f"rope_p{pos}_q"], g[f"rope_p{pos}_k"]
        for rt, name in ((O.ROPE_NORMAL, "normal"), (O.ROPE_NEOX, "neox")):
            gq, gk = orc.rope(q, k, 32, 8, 128, pos0=pos, theta=500000.0, rope_type=rt)
            assert_bits_equal(gq, g[f"rope_p{pos}_{name}_q"], f"q {pos} {name}")
            assert_bits_equal(gk, g[f"rope_p{pos}_{name}_k"], f"k {pos} {name}")


def test_rope_rejects_bad_arguments(orc):
    q = np.zeros((1, 8), np.float32)
    k = np.zeros((1, 4), np.float32)
    for kw in (dict(pos0=-1), dict(theta=0.0), dict(theta=-1.0), dict(theta=float("nan")),
               dict(theta=float("inf"))):
        with pytest.raises(ValueError):
            orc.rope(q, k, 2, 1, 4, **kw)
    with pytest.raises(ValueError):
        orc.rope(np.zeros((1, 6), np.float32), np.zeros((1, 3), np.float32), 2, 1, 3)


# ------------------------------------------------------- silu / softmax

def test_silu_swiglu_closed_forms(orc):
    """test/ops_test.cc:713-725."""
    near(orc.silu(np.array([-2, 0, 2, 1], np.float32)),
         [-2 / (1 + math.exp(2)), 0, 2 / (1 + math.exp(-2)), 1 / (1 + math.exp(-1))])
    near(orc.swiglu(np.array([-2, 0, 2], np.float32), np.array([3, 4, 5], np.float32)),
         [-6 / (1 + math.exp(2)), 0, 10 / (1 + math.exp(-2))])
    g = golden("rows_8b_70b")
    for tag in ("8b", "70b"):
        assert_bits_equal(orc.swiglu(g[f"swiglu_{tag}_g"], g[f"swiglu_{tag}_u"]),
                          g[f"swiglu_{tag}_y"], f"swiglu {tag}")
        assert_bits_equal(orc.silu(g[f"silu_{tag}_x"]), g[f"silu_{tag}_y"], f"silu {tag}")


def test_softmax_closed_form_and_golden(orc):
    g = golden("rows_8b_70b")
    for x, y in ((g["softmax_x"], g["softmax_y"]), (g["softmax_big_x"], g["softmax_big_y"])):
        assert_bits_equal(orc.softmax(x), y, "golden")
        e = np.exp(x.astype(np.float64) - x.max())
        near(orc.softmax(x), e / e.sum(), tol=1e-5)
    d = 1 + math.exp(-1) + math.exp(-2)
    near(orc.softmax(np.array([10000, 9999, 9998], np.float32)), [1 / d, math.exp(-1) / d,
                                                                 math.exp(-2) / d])


# ----------------------------------------------------------- tiny chain

def test_tiny_chain_golden(orc):
    g = golden("tiny_chain")
    H, KV, hd = int(g["n_heads"]), int(g["n_kv_heads"]), int(g["head_dim"])
    assert_bits_equal(orc.gather_f32(g["table"], g["ids"]), g["gathered"], "gather")
    r, y = orc.add_rmsnorm(g["gathered"], g["delta"], g["norm_w"], float(g["eps"]))
    assert_bits_equal(r, g["residual_out"], "residual")
    assert_bits_equal(y, g["norm_out"], "norm")
    q, k = orc.rope(g["q"], g["k"], H, KV, hd, positions=g["positions"], theta=float(g["theta"]))
    assert_bits_equal(q, g["q_out"], "q")
    assert_bits_equal(k, g["k_out"], "k")
    assert_bits_equal(orc.swiglu(g["gate"], g["up"]), g["ffn_out"], "ffn")


def test_chain_baseline_port_matches_ops(orc):
    """The CPU-baseline chain (single thread and ParallelFor) computes what
    the individual ops compute."""
    g = golden("tiny_chain")
    T = len(g["ids"])
    H, KV, hd, F, D = (int(g[k]) for k in ("n_heads", "n_kv_heads", "head_dim", "ffn_dim", "dim"))
    for threads in (1, 2):
        ids = np.tile(g["ids"], 8)  # 48 tokens so ParallelFor splits them over 2 threads
        n = len(ids)
        b = dict(table=g["table"], vocab=int(g["vocab"]), dim=D, ids=ids,
                 x=np.empty((n, D), np.float32), delta=np.tile(g["delta"], (8, 1)),
                 norm_w=g["norm_w"], y=np.empty((n, D), np.float32), eps=float(g["eps"]),
                 q=np.tile(g["q"], (8, 1)), k=np.tile(g["k"], (8, 1)), n_heads=H,
                 n_kv_heads=KV, head_dim=hd, positions=np.tile(g["positions"], 8),
                 theta=float(g["theta"]), gate=np.tile(g["gate"], (8, 1)),
                 up=np.tile(g["up"], (8, 1)), ffn_out=np.empty((n, F), np.float32), ffn_dim=F)
        assert orc.chain(b, n, threads) == 0
        assert_bits_equal(b["y"][:T], g["norm_out"], "y")
        assert_bits_equal(b["y"][-T:], g["norm_out"], "y tail")
        assert_bits_equal(b["q"][-T:], g["q_out"], "q")
        assert_bits_equal(b["ffn_out"][:T], g["ffn_out"], "ffn")


# ------------------------------------------- compiled reference (if built)

needs_ref = pytest.mark.skipif(not O.reference_available(),
                               reason="oracle/_ref is built only where the reference tree exists")


@needs_ref
def test_reference_chain_baselines_match_the_golden_chain(orc):
    """The reference chain the CPU baseline times (the reference's own
    Embedding, ForwardAdd, RmsNorm, Rope, SwiGlu): with a model handle, with
    the table passed per call, and without a gather (the 70B chain: the
    gathered rows given as the residual input), on 1 and 2 threads."""
    ref = O.reference()
    g = golden("tiny_chain")
    T = len(g["ids"])
    H, KV, hd, F, D = (int(g[k]) for k in ("n_heads", "n_kv_heads", "head_dim", "ffn_dim", "dim"))
    model = ref.embedding_model(g["table"])
    try:
        for threads in (1, 2):
            for mode in ("handle", "table", "no_gather"):
                ids = np.tile(g["ids"], 8)
                n = len(ids)
                b = dict(table=g["table"], vocab=int(g["vocab"]), dim=D, ids=ids,
                         x=np.empty((n, D), np.float32), delta=np.tile(g["delta"], (8, 1)),
                         norm_w=g["norm_w"], y=np.empty((n, D), np.float32), eps=float(g["eps"]),
                         q=np.tile(g["q"], (8, 1)), k=np.tile(g["k"], (8, 1)), n_heads=H,
                         n_kv_heads=KV, head_dim=hd, positions=np.tile(g["positions"], 8),
                         theta=float(g["theta"]), gate=np.tile(g["gate"], (8, 1)),
                         up=np.tile(g["up"], (8, 1)), ffn_out=np.empty((n, F), np.float32),
                         ffn_dim=F)
                if mode == "handle":
                    b["model"] = model
                elif mode == "no_gather":
                    b["table"] = None
                    b["x_in"] = np.tile(g["gathered"], (8, 1))
                assert ref.chain(b, n, threads) == 0, mode
                assert_bits_equal(b["x"][-T:], g["residual_out"], mode + " residual")
                assert_bits_equal(b["y"][:T], g["norm_out"], mode + " y")
                assert_bits_equal(b["q"][-T:], g["q_out"], mode + " q")
                assert_bits_equal(b["k"][:T], g["k_out"], mode + " k")
                assert_bits_equal(b["ffn_out"][-T:], g["ffn_out"], mode + " ffn")
    finally:
        ref.free_model(model)


@needs_ref
def test_reference_quantized_gather_baseline_matches_the_oracle(orc):
    ref = O.reference()
    rng = np.random.default_rng(5)
    table = (rng.standard_normal((50, 96)) * 0.02).astype(np.float32)
    ids = rng.integers(0, 50, 40).astype(np.int32)
    for qt in QT:
        blocks = orc.quantize(qt, table)
        want = orc.gather_quant(qt, blocks, 50, 96, ids)
        for threads in (1, 2):
            assert_bits_equal(ref.gather_quant(qt, blocks, 50, 96, ids, threads), want, qt)


@needs_ref
def test_oracle_equals_compiled_reference_on_random_inputs(orc):
    ref = O.reference()
    rng = np.random.default_rng(11)
    for qt in QT:
        for cols in (1, 31, 32, 33, 100, 4096):
            x = (rng.standard_normal((3, cols)) * rng.choice([1e-4, 0.02, 3.0])).astype(np.float32)
            a = orc.quantize(qt, x)
            np.testing.assert_array_equal(a, ref.quantize(qt, x))
            assert_bits_equal(orc.dequantize(qt, a, 3, cols), ref.dequantize(qt, a, 3, cols), qt)
    for dim in (1, 7, 4096, 8192):
        x = rng.standard_normal(dim).astype(np.float32)
        w = rng.standard_normal(dim).astype(np.float32)
        assert_bits_equal(orc.rmsnorm(x, w, 1e-5), ref.rmsnorm_row(x, w, 1e-5), "rms")
    for hd, pos, theta in ((8, 63, 1e4), (128, 8191, 5e5), (130, 7, 1e4), (2, 3, 100.0)):
        q = rng.standard_normal((1, 5 * hd)).astype(np.float32)
        k = rng.standard_normal((1, 2 * hd)).astype(np.float32)
        for rt in (O.ROPE_NORMAL, O.ROPE_NEOX):
            gq, gk = orc.rope(q, k, 5, 2, hd, pos0=pos, theta=theta, rope_type=rt)
            rq, rk = ref.rope_token(q, k, 5, 2, hd, pos, theta, rt)
            assert_bits_equal(gq, rq, "q")
            assert_bits_equal(gk, rk, "k")
    g = (rng.standard_normal(5000) * 4).astype(np.float32)
    u = rng.standard_normal(5000).astype(np.float32)
    assert_bits_equal(orc.swiglu(g, u), ref.swiglu(g, u), "swiglu")
    assert_bits_equal(orc.softmax(g), ref.softmax(g), "softmax")


# ----------------------------------------------------- planted mistakes

def _rope_mutant(q, pos, theta, mutation):
    """float64 Normal RoPE of one head with a planted mistake."""
    hd = q.size
    out = q.astype(np.float64).copy()
    for i in range(hd // 2):
        a = pos * theta ** (-2.0 * i / hd)
        c, s = math.cos(a), math.sin(a)
        if mutation == "sign":
            s = -s
        x0, x1 = q[2 * i], q[2 * i + 1]
        if mutation == "index":
            x0, x1 = x1, x0
        out[2 * i] = x0 * c - (0 if mutation == "drop" else x1 * s)
        out[2 * i + 1] = x0 * s + x1 * c
    return out


@pytest.mark.parametrize("mutation", ["sign", "index", "drop"])
def test_planted_rope_mistakes_fail_the_kat(mutation):
    q = np.array([1, 2, 3, 4], np.float64)
    assert np.allclose(_rope_mutant(q, 1, 100.0, "none"), KAT_NORMAL[0], atol=1e-12)
    with pytest.raises(AssertionError):
        near(_rope_mutant(q, 1, 100.0, mutation), KAT_NORMAL[0])


@pytest.mark.parametrize("mutation", ["mean_not_sum", "no_eps", "weight_index"])
def test_planted_rmsnorm_mistakes_fail_the_kat(mutation):
    x = np.array([-2, 0.25, 3.5])
    w = np.array([0.5, 2, -1])
    eps = 1e-2  # large enough that dropping it is visible
    ss = np.sum(x * x) * (x.size if mutation == "mean_not_sum" else 1)
    den = math.sqrt(ss / x.size + (0 if mutation == "no_eps" else eps))
    ww = w[::-1] if mutation == "weight_index" else w
    with pytest.raises(AssertionError):
        near(x / den * ww, rms_closed_form(x, w, eps))


def test_planted_q4_nibble_swap_fails_the_kat(orc):
    q40 = np.zeros(18, np.uint8)
    q40[0:2] = [0x00, 0x38]
    i = np.arange(16)
    q40[2:] = ((15 - i) << 4) | i
    right = orc.dequantize("q4_0", q40, 1, 32)[0]
    swapped = np.concatenate([right[16:], right[:16]])  # high nibble read as the first 16
    assert not np.array_equal(swapped[:16], 0.5 * (i - 8))


# ------------------------------------------------------------------- linear

U = 2.0 ** -24  # unit roundoff of float32


def gamma(n):
    """Higham, Accuracy and Stability of Numerical Algorithms, eq. 3.8: a
    recursive fp32 dot product of n terms is within gamma_n * sum|x_k w_k| of
    the exact value, in any summation order."""
    return n * U / (1 - n * U)


def linear_exact(x, w, bias=None):
    """float64 value and sum of |terms| of x @ w^T (+ bias)."""
    x64, w64 = np.asarray(x, np.float64), np.asarray(w, np.float64)
    y = np.atleast_2d(x64) @ w64.T
    s = np.abs(np.atleast_2d(x64)) @ np.abs(w64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
        s = s + np.abs(np.asarray(bias, np.float64))
    return y, s


def within_dot_bound(got, exact, abs_terms, n):
    got = np.atleast_2d(np.asarray(got, np.float64))
    return bool((np.abs(got - exact) <= gamma(n) * abs_terms + 1e-30).all())


def test_linear_quant_golden(orc):
    """LinearQ80/Q40/Q41 of the reference's default build, bit for bit."""
    g = golden("linear")
    n = 0
    for key in list(g):
        if not key.endswith("_w") or key.startswith("f32"):
            continue
        tag = key[:-2]
        qt = next(q for q in QT if f"_{q}_" in tag)
        for xk in [k for k in g if k.startswith(tag + "_x")]:
            yk = tag + "_y" + xk[len(tag) + 2:]
            x, y = g[xk], g[yk]
            got = orc.linear_quant(qt, x, g[key], y.shape[-1])
            assert_bits_equal(got, y, yk)
            n += 1
    assert n == 3 * (5 * 2 + 2 + 2)


@pytest.mark.parametrize("qt", QT)
def test_linear_quant_float64_closed_form(orc, qt):
    """Within the recursive-summation bound of the float64 value of the
    dequantized product, and within test/cuda_quant_test.cc:60-66's
    2e-5 * max(1, |y|) on that test's own inputs and shapes."""
    g = golden("linear")
    for inf in (1, 17, 32, 33, 65):
        blocks = g[f"p43_{qt}_{inf}_w"]
        w = orc.dequantize(qt, blocks, 131, inf)
        for rows in (1, 3):
            x = g[f"p43_{qt}_{inf}_x{rows}"]
            bias = g["sin_bias7"][0] * np.ones(131, np.float32)
            got = orc.linear_quant(qt, x, blocks, 131, bias=bias)
            ex, s = linear_exact(x, w, bias)
            assert within_dot_bound(got, ex, s, inf + 1)
            near(got, ex)
    rng = np.random.default_rng(3)
    for out_f, inf in ((9, 4096), (3, 14336), (5, 70)):
        w = (rng.standard_normal((out_f, inf)) * 0.02).astype(np.float32)
        blocks = orc.quantize(qt, w)
        x = rng.standard_normal((2, inf)).astype(np.float32)
        ex, s = linear_exact(x, orc.dequantize(qt, blocks, out_f, inf))
        assert within_dot_bound(orc.linear_quant(qt, x, blocks, out_f), ex, s, inf)


def test_linear_f32_and_matmul(orc):
    g = golden("linear")
    assert_bits_equal(orc.linear_f32(g["f32_x"], g["f32_w"]), g["f32_y"], "linear f32")
    got = orc.linear_f32(g["f32_x"], g["f32_w"], bias=g["f32_bias"])
    assert_bits_equal(got, g["f32_y"] + g["f32_bias"], "bias is one fp32 add after the sum")
    for m, k, n in ((3, 7, 5), (1, 33, 17)):
        a, b = g[f"mm_{m}x{k}x{n}_a"], g[f"mm_{m}x{k}x{n}_b"]
        c = orc.matmul_f32(a, b)
        assert_bits_equal(c, g[f"mm_{m}x{k}x{n}_c"], "matmul")
        ex, s = linear_exact(a, b.T)
        assert within_dot_bound(c, ex, s, k)
    # Linear(x, W) == Matmul(x, W^T)
    x, w = g["f32_x"], g["f32_w"]
    assert_bits_equal(orc.linear_f32(x, w), orc.matmul_f32(x, np.ascontiguousarray(w.T)), "lin")


def test_linear_threads_do_not_change_results_and_bad_shapes_raise(orc):
    rng = np.random.default_rng(8)
    w = rng.standard_normal((200, 96)).astype(np.float32)
    x = rng.standard_normal((4, 96)).astype(np.float32)
    blocks = orc.quantize("q4_1", w)
    one = orc.linear_quant("q4_1", x, blocks, 200, n_threads=1)
    assert_bits_equal(orc.linear_quant("q4_1", x, blocks, 200, n_threads=7), one, "threads")
    assert_bits_equal(orc.linear_f32(x, w, n_threads=5), orc.linear_f32(x, w, n_threads=1), "f")
    with pytest.raises(ValueError):
        orc.linear_quant("q8_0", np.zeros((0, 96), np.float32), blocks, 200)
    with pytest.raises(ValueError):
        orc.matmul_f32(np.zeros((2, 0), np.float32), np.zeros((0, 3), np.float32))


@pytest.mark.parametrize("mutation", ["neighbour_scale", "nibble_swap", "drop_min", "k_reversed"])
def test_planted_linear_mistakes_fail_the_closed_form(orc, mutation):
    """A copy of the quantized dot product with one planted mistake, checked
    like the oracle is: it fails the float64 bound on the golden inputs."""
    g = golden("linear")
    qt = "q4_1" if mutation == "drop_min" else ("q4_0" if mutation == "nibble_swap" else "q8_0")
    blocks, x = g[f"n_{qt}_32x4096_w"], g[f"n_{qt}_32x4096_x"]
    w = orc.dequantize(qt, blocks, 32, 4096).astype(np.float64)
    wb = w.reshape(32, 128, 32)
    if mutation == "neighbour_scale":
        ratio = np.abs(wb).max(-1, keepdims=True)
        wb = wb / np.maximum(ratio, 1e-30) * np.roll(ratio, 1, axis=1)
    elif mutation == "nibble_swap":
        wb = np.concatenate([wb[..., 16:], wb[..., :16]], axis=-1)
    elif mutation == "drop_min":
        raw = blocks.reshape(32, 128, 20)
        mins = orc.fp16_to_fp32_array(raw[..., 2:4].copy().view(np.uint16)[..., 0])
        wb = wb - mins[..., None]
    else:
        wb = wb[..., ::-1]
    wrong = x.astype(np.float64) @ wb.reshape(32, 4096).T
    ex, s = linear_exact(x, w)
    assert within_dot_bound(g[f"n_{qt}_32x4096_y"], ex, s, 4096)
    assert not within_dot_bound(wrong, ex, s, 4096)


@needs_ref
def test_linear_oracle_equals_compiled_reference_on_random_inputs(orc):
    ref = O.reference()
    rng = np.random.default_rng(12)
    for qt in QT:
        for out_f, inf, rows in ((131, 65, 3), (7, 32, 1), (40, 4096, 2), (33, 1, 2)):
            w = (rng.standard_normal((out_f, inf)) * 0.3).astype(np.float32)
            blocks = orc.quantize(qt, w)
            x = rng.standard_normal((rows, inf)).astype(np.float32)
            assert_bits_equal(orc.linear_quant(qt, x, blocks, out_f),
                              ref.linear_quant(qt, x, blocks, out_f), qt)
    w = rng.standard_normal((50, 300)).astype(np.float32)
    x = rng.standard_normal((3, 300)).astype(np.float32)
    assert_bits_equal(orc.linear_f32(x, w), ref.linear_f32(x, w), "f32")
    a = rng.standard_normal((6, 40)).astype(np.float32)
    assert_bits_equal(orc.matmul_f32(a, w[:40, :9].copy()), ref.matmul_f32(a, w[:40, :9].copy()),
                      "mm")


# ------------------------------------------------- attention, KV cache

def attention_f64(q, k, v, pos, kv_of=None, scale=None, last=None, values=None):
    """test/cuda_attention_test.cc:50-80: float64 scores q.k / sqrt(hd),
    softmax and value sums over positions 0..pos.  q [H, hd], k / v
    [>= pos + 1, KV, hd].  The keyword arguments plant mistakes (for the
    planted-mistake test): another query-to-KV-head map, scale, last
    attended position, or the rows the values come from."""
    H, hd = q.shape
    KV = k.shape[1]
    group = H // KV
    kv_of = kv_of or (lambda h: h // group)
    scale = 1.0 / math.sqrt(hd) if scale is None else scale
    last = pos if last is None else last
    values = v if values is None else values
    out = np.empty((H, hd))
    for h in range(H):
        kk = k[:last + 1, kv_of(h)].astype(np.float64)
        s = kk @ q[h].astype(np.float64) * scale
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ values[:last + 1, kv_of(h)].astype(np.float64)
    return out


def cache_from_rows(orc, k_rows, v_rows, n_layers, max_seq, layer):
    L, S = int(n_layers), int(max_seq)
    KV, hd = k_rows.shape[1], k_rows.shape[2]
    kc = np.zeros((L, S, KV, hd), np.float32)
    vc = np.zeros_like(kc)
    n = k_rows.shape[0]
    orc.kv_write(kc, vc, layer, np.arange(n), k_rows, v_rows)
    return kc, vc


ATT_CASES = ("c0", "c1", "c2", "g")


@pytest.mark.parametrize("case", ATT_CASES)
def test_attention_golden_and_closed_form(orc, case):
    """Golden outputs of the compiled reference (bit for bit) and the
    float64 closed form of the reference's own GPU test within its 2e-5."""
    g = golden("attention")
    H, KV, hd, pos, layer, L, S = (int(v) for v in g[f"{case}_shape"])
    q, k, v = g[f"{case}_q"], g[f"{case}_k"], g[f"{case}_v"]
    kc, vc = cache_from_rows(orc, k, v, L, S, layer)
    got = orc.attention(q[None], kc, vc, layer, [pos])[0]
    assert_bits_equal(got, g[f"{case}_out"], case)
    near(got, attention_f64(q, k, v, pos))


def test_attention_invariants(orc):
    rng = np.random.default_rng(31)
    H, KV, hd, S = 8, 2, 32, 40
    q = rng.standard_normal((H, hd)).astype(np.float32)
    k = rng.standard_normal((S, KV, hd)).astype(np.float32)
    v = rng.standard_normal((S, KV, hd)).astype(np.float32)
    kc, vc = cache_from_rows(orc, k, v, 1, S, 0)
    # pos 0: one score, softmax 1, the output is the value row itself
    out0 = orc.attention(q[None], kc, vc, 0, [0])[0]
    assert_bits_equal(out0, np.repeat(v[0], H // KV, axis=0), "pos 0")
    # slots after pos take no part
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[0, 21:] = 1e30
    vc2[0, 21:] = np.nan
    assert_bits_equal(orc.attention(q[None], kc2, vc2, 0, [20]),
                      orc.attention(q[None], kc, vc, 0, [20]), "future slots")
    # equal keys: uniform weights, the output is the mean value row
    kc3 = np.broadcast_to(kc[:, :1], kc.shape).copy()
    out = orc.attention(q[None], kc3, vc, 0, [S - 1])[0]
    near(out, np.repeat(v.astype(np.float64).mean(axis=0), H // KV, axis=0), tol=1e-6)
    # GQA: query head h reads KV head h // (H / KV)
    vc4 = np.zeros_like(vc)
    vc4[0, :, 1] = 1.0
    out = orc.attention(q[None], kc, vc4, 0, [S - 1])[0]
    near(out[:, 0], (np.arange(H) // (H // KV)).astype(np.float64), tol=1e-6)
    # several tokens at once equal one call per token
    pos = np.array([3, 39, 0, 17], np.int32)
    qs = rng.standard_normal((4, H, hd)).astype(np.float32)
    batch = orc.attention(qs, kc, vc, 0, pos)
    for t in range(4):
        assert_bits_equal(batch[t], orc.attention(qs[t:t + 1], kc, vc, 0, pos[t:t + 1])[0], "t")


def test_kv_write_slots_and_rejections(orc):
    rng = np.random.default_rng(32)
    L, S, KV, hd = 3, 9, 2, 5
    kc = rng.standard_normal((L, S, KV, hd)).astype(np.float32)
    vc = rng.standard_normal((L, S, KV, hd)).astype(np.float32)
    before_k, before_v = kc.copy(), vc.copy()
    pos = np.array([4, 0, 8], np.int32)
    k = rng.standard_normal((3, KV, hd)).astype(np.float32)
    v = rng.standard_normal((3, KV, hd)).astype(np.float32)
    orc.kv_write(kc, vc, 2, pos, k, v)
    want_k, want_v = before_k.copy(), before_v.copy()
    want_k[2, pos], want_v[2, pos] = k, v
    assert_bits_equal(kc, want_k, "k slots")
    assert_bits_equal(vc, want_v, "v slots")
    for layer, p in ((3, [0]), (-1, [0]), (0, [9]), (0, [-1])):
        with pytest.raises(ValueError):
            orc.kv_write(kc, vc, layer, np.array(p, np.int32), k[:1], v[:1])
    with pytest.raises(ValueError):
        orc.attention(np.zeros((1, 3, hd), np.float32), kc, vc, 0, [0])  # 3 % 2 != 0


@pytest.mark.parametrize("mutation", ["kv_head_mod", "no_scale", "drop_last", "values_from_k"])
def test_planted_attention_mistakes_fail_the_golden(mutation):
    g = golden("attention")
    q, k, v = g["g_q"], g["g_k"], g["g_v"]
    H, KV, hd, pos = (int(x) for x in g["g_shape"][:4])
    kw = {"kv_head_mod": dict(kv_of=lambda h: h % KV), "no_scale": dict(scale=1.0),
          "drop_last": dict(last=pos - 1), "values_from_k": dict(values=k)}[mutation]
    ref_out = g["g_out"].astype(np.float64)
    assert np.abs(attention_f64(q, k, v, pos) - ref_out).max() <= 2e-5
    assert np.abs(attention_f64(q, k, v, pos, **kw) - ref_out).max() > 2e-5


@needs_ref
def test_attention_oracle_equals_compiled_reference_on_random_inputs(orc):
    ref = O.reference()
    rng = np.random.default_rng(33)
    for H, KV, hd, pos in ((32, 8, 128, 200), (6, 3, 17, 9), (4, 4, 64, 0), (8, 1, 96, 77)):
        q = rng.standard_normal((H, hd)).astype(np.float32)
        k = rng.standard_normal((pos + 1, KV, hd)).astype(np.float32)
        v = rng.standard_normal((pos + 1, KV, hd)).astype(np.float32)
        kc, vc = cache_from_rows(orc, k, v, 2, pos + 3, 1)
        assert_bits_equal(orc.attention(q[None], kc, vc, 1, [pos])[0],
                          ref.attention(q, k, v, 2, pos + 3, 1, pos), f"{H}/{KV}/{hd}/{pos}")


# ------------------------------------------------------------ forward pass

from conftest import tiny_model  # noqa: E402


def test_forward_tokens_matches_reference_tiny_model(orc):
    """The restated ForwardToken loop reproduces the reference's own CPU
    forward pass on its tiny model bit for bit (tests/golden/tiny_forward)."""
    model, tokens, positions, logits = tiny_model()
    got, hidden = orc.forward_tokens(model, tokens, positions)
    assert_bits_equal(got, logits, "tiny model logits")
    assert_bits_equal(hidden[:, 0], model["embedding"][tokens], "layer 0 input = embedding row")


@pytest.mark.parametrize("mistake", O.FORWARD_MISTAKES)
def test_forward_tokens_planted_mistakes_fail(orc, mistake):
    """Each planted wiring mistake moves the logits of a random GQA model
    (norm weights N(1, 0.1): the tiny model's are all 1, so a swap of its two
    norms would not show) away from the pinned result."""
    cfg = dict(vocab=131, dim=64, hidden_dim=100, layers=2, n_heads=4, n_kv_heads=2,
               head_dim=16, max_seq=32, rope_type=0, theta=10000.0, eps=1e-5)
    model = O.forward_model(cfg, seed=5, biases=True)
    tokens, positions = np.array([1, 7, 99, 3, 60], np.int32), np.arange(5, dtype=np.int32)
    want, _ = orc.forward_tokens(model, tokens, positions)
    if O.reference_available():
        assert_bits_equal(want, O.reference().forward_tokens(model, tokens, positions), "pin")
    got, _ = orc.forward_tokens(model, tokens, positions, mistake=mistake)
    assert np.abs(got - want).max() > 1e-4, mistake


def test_forward_tokens_zero_blocks_keep_the_embedding(orc):
    """Closed form of the wiring: with wo and w_down zero, both residual
    adds add zero, so every layer passes the embedding row through and the
    logits are lm_head . RmsNorm(embedding row)."""
    model, tokens, positions, _ = tiny_model()
    for lw in model["layers"]:
        lw["wo"] = ("f32", np.zeros_like(lw["wo"][1]))
        lw["w_down"] = ("f32", np.zeros_like(lw["w_down"][1]))
    got, hidden = orc.forward_tokens(model, tokens, positions)
    emb = model["embedding"][tokens]
    for li in range(hidden.shape[1]):
        assert_bits_equal(hidden[:, li], emb, f"residual stream at {li}")
    c = model["config"]
    want = orc.linear_f32(orc.rmsnorm(emb, model["final_norm"], c["eps"]), model["lm_head"][1])
    assert_bits_equal(got, want, "logits")


FORWARD_CASES = [  # config overrides, weight type, biases, positions
    (dict(), "f32", False, "contiguous"),
    (dict(n_kv_heads=2, head_dim=64, dim=128, hidden_dim=200), "q8_0", True, "contiguous"),
    (dict(n_kv_heads=1, rope_type=1), "q4_0", False, "gaps"),
    (dict(n_heads=6, n_kv_heads=3, head_dim=16, dim=96, layers=3), "q4_1", True, "contiguous"),
]


@needs_ref
@pytest.mark.parametrize("over,wt,biases,pos_kind", FORWARD_CASES)
def test_forward_tokens_matches_compiled_reference(orc, over, wt, biases, pos_kind):
    """GQA / MQA / NeoX, quantized weights, q/k/v biases and increasing
    positions with gaps: bit-identical to the compiled ForwardToken loop."""
    cfg = dict(vocab=131, dim=32, hidden_dim=86, layers=2, n_heads=4, n_kv_heads=4, head_dim=8,
               max_seq=64, rope_type=0, theta=10000.0, eps=1e-5)
    cfg.update(over)
    model = O.forward_model(cfg, seed=len(over) + 3, weight_type=wt, biases=biases)
    tokens = np.array([5, 9, 100, 3, 7, 8, 64, 1, 2, 130], np.int32)
    positions = (np.arange(10) if pos_kind == "contiguous"
                 else np.array([0, 1, 3, 4, 9, 10, 11, 20, 21, 40])).astype(np.int32)
    got, _ = orc.forward_tokens(model, tokens, positions)
    assert_bits_equal(got, O.reference().forward_tokens(model, tokens, positions), "logits")
