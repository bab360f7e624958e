"""GPU parity of the batched forward pass (mlk_forward_layer_batch through
cpp_minilamma_amd.forward.DeviceModel): the reference's ForwardBatch without
its token loop.

The bar is the reference's own for its device forward pass against its CPU
one: |got - want| <= 1e-5 + 1e-4 |want| on every logit
(test/forward_test.cc:276-285).  `want` is the reference's CPU forward
pass: its own logits on its tiny model (tests/golden/tiny_forward.npz,
written by the compiled reference), and elsewhere the oracle's restatement
of the ForwardToken loop, which equals the compiled reference bit for bit
(tests/test_oracle.py).  The reference's batch tests are mirrored: one batch
equals prefill + single decode steps equals token by token
(test/forward_test.cc:118-183).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from conftest import U32, assert_bits_equal, tiny_model

pytestmark = pytest.mark.gpu


def assert_forward_close(got, want, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert np.isfinite(got).all(), f"{what}: non-finite"
    err = np.abs(got - want)
    lim = 1e-5 + 1e-4 * np.abs(want)
    bad = err > lim
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {got.size} logits outside "
                           f"1e-5 + 1e-4|x|; worst err {float(err.max()):.3e}")


@pytest.fixture(scope="module")
def fwd(mlk):
    import importlib
    return importlib.import_module(mlk.__name__ + ".forward")


def test_tiny_model_batch_matches_reference(fwd):
    """The reference's tiny model: the whole 9-token prompt as one batch
    (GEMM linears, decode attention at head_dim 8) gives the logits the
    reference's CPU forward pass gives for each token."""
    model, tokens, positions, logits = tiny_model()
    dm = fwd.DeviceModel(model)
    got = dm.forward(tokens, pos0=0, all_logits=True)
    assert_forward_close(got, logits, "batch of 9")


def test_tiny_model_prefill_then_decode_and_token_by_token(fwd):
    """test/forward_test.cc:118-183: a prefill batch followed by single
    decode tokens, and every token alone, give the same logits."""
    model, tokens, positions, logits = tiny_model()
    dm = fwd.DeviceModel(model)
    got = dm.forward(tokens[:6], pos0=0, all_logits=True)
    assert_forward_close(got, logits[:6], "prefill of 6")
    for t in range(6, len(tokens)):
        assert_forward_close(dm.forward(tokens[t:t + 1], pos0=t), logits[t], f"decode {t}")
    single = fwd.DeviceModel(model)
    for t in range(len(tokens)):
        assert_forward_close(single.forward(tokens[t:t + 1], pos0=t), logits[t], f"token {t}")


CASES = [  # config overrides, weight type, biases, tokens in the prefill batch
    (dict(dim=256, hidden_dim=512, n_heads=4, n_kv_heads=2, head_dim=64), "f32", True, 40),
    (dict(dim=256, hidden_dim=512, n_heads=4, n_kv_heads=2, head_dim=64), "q8_0", True, 40),
    (dict(dim=512, hidden_dim=768, n_heads=4, n_kv_heads=1, head_dim=128), "q4_0", False, 33),
    (dict(dim=256, hidden_dim=384, n_heads=8, n_kv_heads=2, head_dim=32, rope_type=1), "q4_1",
     True, 20),
    (dict(dim=512, hidden_dim=1024, n_heads=8, n_kv_heads=8, head_dim=64, layers=3), "q8_0",
     False, 64),
]


@pytest.mark.parametrize("over,wt,biases,T", CASES)
def test_forward_batch_matches_oracle(orc, fwd, over, wt, biases, T):
    """Random models (GQA, MQA, MHA; NeoX; head_dim 32 / 64 / 128 so both
    attention kernels run; every weight type; q/k/v biases): a prefill batch
    of T tokens, then 3 single decode tokens, against the reference's
    ForwardToken loop over the same tokens."""
    cfg = dict(vocab=300, layers=2, max_seq=128, rope_type=0, theta=10000.0, eps=1e-5)
    cfg.update(over)
    model = O.forward_model(cfg, seed=T + len(over), weight_type=wt, biases=biases)
    rng = np.random.default_rng(T)
    tokens = rng.integers(0, cfg["vocab"], T + 3).astype(np.int32)
    positions = np.arange(T + 3, dtype=np.int32)
    want, hidden = orc.forward_tokens(model, tokens, positions)
    dm = fwd.DeviceModel(model)
    x = dm.hidden(tokens[:T], pos0=0)
    np.testing.assert_allclose(x.download(), hidden[:T, -1], rtol=1e-4, atol=1e-5,
                               err_msg="residual stream after the last layer")
    got = dm.logits(x, T).download()
    assert_forward_close(got, want[:T], f"prefill {wt}")
    for t in range(T, T + 3):
        assert_forward_close(dm.forward(tokens[t:t + 1], pos0=t), want[t], f"decode {t}")


def test_forward_batch_positions_with_gaps(orc, fwd):
    """Increasing positions with gaps (the device positions array: RoPE,
    cache slots and the decode attention kernel read it): equal to the token
    loop at the same positions."""
    cfg = dict(vocab=200, dim=256, hidden_dim=384, layers=2, n_heads=4, n_kv_heads=2,
               head_dim=64, max_seq=256, rope_type=0, theta=10000.0, eps=1e-5)
    model = O.forward_model(cfg, seed=3, weight_type="q8_0", biases=True)
    tokens = np.arange(1, 25, dtype=np.int32) * 7 % 200
    positions = np.cumsum(np.arange(1, 25) % 4 + 1).astype(np.int32) - 2
    want, _ = orc.forward_tokens(model, tokens, positions)
    dm = fwd.DeviceModel(model)
    got = dm.logits(dm.hidden(tokens, positions=positions), len(tokens)).download()
    assert_forward_close(got, want, "gapped positions")


@pytest.mark.parametrize("qt", ["q8_0", "q4_0", "q4_1"])
def test_forward_batch_quantized_token_table(orc, fwd, qt):
    """The token table kept as GGUF-style blocks on the device and gathered
    from them (the reference dequantizes it at load): same logits as the
    token loop over the dequantized table."""
    cfg = dict(vocab=257, dim=256, hidden_dim=384, layers=2, n_heads=4, n_kv_heads=2,
               head_dim=64, max_seq=64, rope_type=0, theta=10000.0, eps=1e-5)
    model = O.forward_model(cfg, seed=9, weight_type=qt, quant_embedding=qt)
    tokens = np.array([256, 0, 17, 3, 200, 99, 5, 5, 8, 1, 2, 3, 4, 128, 64, 32, 1, 0],
                      np.int32)
    positions = np.arange(tokens.size, dtype=np.int32)
    want, _ = orc.forward_tokens(model, tokens, positions)
    dm = fwd.DeviceModel(model)
    got = dm.forward(tokens, pos0=0, all_logits=True)
    assert_forward_close(got, want, f"{qt} token table")


def test_forward_layer_rejects(mlk, fwd):
    cfg = dict(dim=64, hidden_dim=128, n_heads=4, n_kv_heads=3, head_dim=16, theta=1e4,
               eps=1e-5)
    w = fwd.LayerWeights()
    x = mlk.DeviceBuffer.empty((4, 64))
    kc = mlk.DeviceBuffer.empty((1, 16, 3, 16))
    ws = mlk.DeviceBuffer(1 << 20, np.uint8)
    with pytest.raises(mlk.MlkError, match="divide n_heads"):
        fwd.forward_layer_batch(cfg, w, x, 4, kc, kc, 1, 16, 0, 16, ws)
    cfg["n_kv_heads"] = 2
    with pytest.raises(mlk.MlkError, match="norm weights"):
        fwd.forward_layer_batch(cfg, w, x, 4, kc, kc, 1, 16, 0, 16, ws)


def test_forward_layer_rejects_cache_arguments(mlk, fwd):
    """The layer checks the caches before its first launch: the fused q/k/v
    launch writes cache rows directly, so a bad layer index or a shared
    K/V buffer must never reach a kernel."""
    cfg = dict(vocab=64, dim=512, hidden_dim=1536, layers=1, n_heads=8, n_kv_heads=2,
               head_dim=64, max_seq=32, rope_type=0, theta=10000.0, eps=1e-5)
    model = O.forward_model(cfg, seed=2, weight_type="q8_0")
    dm = fwd.DeviceModel(model)
    x = mlk.DeviceBuffer.empty((1, 512))
    kc, vc = mlk.DeviceBuffer.empty((1, 32, 2, 64)), mlk.DeviceBuffer.empty((1, 32, 2, 64))
    ws = mlk.DeviceBuffer(fwd.layer_workspace_bytes(cfg, 1, 32, True), np.uint8)
    with pytest.raises(mlk.MlkError, match="layer 1 out of range"):
        fwd.forward_layer_batch(cfg, dm.layers[0], x, 1, kc, vc, 1, 32, 1, 32, ws, pos0=3)
    with pytest.raises(mlk.MlkError, match="distinct"):
        fwd.forward_layer_batch(cfg, dm.layers[0], x, 1, kc, kc, 1, 32, 0, 32, ws, pos0=3)
    with pytest.raises(mlk.MlkError, match="out of range"):
        fwd.forward_layer_batch(cfg, dm.layers[0], x, 1, kc, vc, 1, 32, 0, 32, ws, pos0=-1)
    # the NeoX layout and F32 weights keep the separate RoPE and q/k/v
    # launches: a negative position is still rejected before the first one
    for rope_type, wt, T in ((1, "q8_0", 1), (0, "f32", 1), (0, "q8_0", 2)):
        c2 = dict(cfg, rope_type=rope_type)
        m2 = O.forward_model(c2, seed=3, weight_type=wt)
        d2 = fwd.DeviceModel(m2)
        x2 = mlk.DeviceBuffer.empty((T, 512))
        before = x2.download()
        ws2 = mlk.DeviceBuffer(fwd.layer_workspace_bytes(c2, T, 32, True), np.uint8)
        with pytest.raises(mlk.MlkError, match="out of range"):
            fwd.forward_layer_batch(c2, d2.layers[0], x2, T, kc, vc, 1, 32, 0, 32, ws2, pos0=-1)
        mlk.synchronize()
        assert_bits_equal(x2.download(), before, f"x untouched (rope {rope_type}, {wt}, T {T})")


@pytest.mark.parametrize("wt", ["q8_0", "q4_0", "q4_1", "f32"])
@pytest.mark.parametrize("T", [1, 12, 24, 40])
@pytest.mark.parametrize("case", ["pos0", "positions", "bad_position", "neox"])
def test_layer_fused_equals_op_by_op(mlk, fwd, wt, T, case):
    """One token (streaming GEMVs) and 8..32 tokens (skinny GEMMs) through a
    layer with quantized weights take fused launches: q/k/v in one, which
    also rotates q and k (normal layout) and writes k and v into the cache,
    gate/up with the SwiGLU epilogue, down adding into x (for 8..32 tokens
    the epilogues run in the split-K reduction).  Their per-element
    arithmetic is the separate ops', so the layer equals the same layer
    composed from the individual entry points bit for bit (residual stream,
    K/V cache rows, error flag).  Cases: consecutive positions from pos0 (24
    tokens also take the prefill attention kernel); scattered positions;
    one position at max_seq (flagged, its cache row not written, its
    attention output zero); the NeoX layout (separate RoPE and K/V write).
    The cache spans several attention chunks, so the decode attention's
    in-kernel merge of them (after the fused q/k/v launch) is compared with
    the separate merge launch.  40 tokens (and F32 weights from 8 rows) take
    the matrix-core GEMM and the separate SwiGLU and residual-add launches."""
    S = 1024
    cfg = dict(vocab=64, dim=512, hidden_dim=1536, layers=1, n_heads=8, n_kv_heads=2,
               head_dim=64, max_seq=S, rope_type=1 if case == "neox" else 0, theta=10000.0,
               eps=1e-5)
    model = O.forward_model(cfg, seed=11, weight_type=wt, biases=True)
    D, F, H, KV, hd = 512, 1536, 8, 2, 64
    QD, KD, pos = H * hd, KV * hd, 700
    lw = model["layers"][0]
    dm = fwd.DeviceModel(model)
    rng = np.random.default_rng(5)
    x0 = rng.standard_normal((T, D)).astype(np.float32)
    kc0 = (rng.standard_normal((1, S, KV, hd)) * 0.5).astype(np.float32)
    vc0 = rng.standard_normal((1, S, KV, hd)).astype(np.float32)
    B = mlk.DeviceBuffer.from_array
    positions = None
    if case in ("positions", "bad_position"):
        pv = np.sort(rng.choice(S, T, replace=False)).astype(np.int32)
        if case == "bad_position":
            pv[T // 2] = S
        positions = B(pv)
    contiguous = positions is None
    flag, flag2 = B(np.zeros(1, np.int32)), B(np.zeros(1, np.int32))

    # fused: the layer entry point
    x = B(x0)
    kc, vc = B(kc0), B(vc0)
    ws = mlk.DeviceBuffer(fwd.layer_workspace_bytes(cfg, T, S, contiguous), np.uint8)
    fwd.forward_layer_batch(cfg, dm.layers[0], x, T, kc, vc, 1, S, 0, S, ws, positions=positions,
                            pos0=pos, err=flag)
    got = x.download()

    # the same layer op by op
    def up(a):
        return B(np.ascontiguousarray(a))
    w = {n: up(np.asarray(lw[n][1], np.float32 if wt == "f32" else np.uint8))
         for n in fwd.LINEAR_NAMES}
    bias = {n: up(np.asarray(lw["b" + n[1]], np.float32)) for n in ("wq", "wk", "wv")}
    an, fn = up(np.asarray(lw["attention_norm"], np.float32)), up(np.asarray(lw["ffn_norm"], np.float32))
    x2, kc2, vc2 = B(x0), B(kc0), B(vc0)

    def linear(name, x_in, y_out, rows, i, o, b=None):
        if wt == "f32":
            mlk.linear_f32(x_in, w[name], y_out, rows, i, o, bias=b)
        else:
            mlk.linear_quant(wt, x_in, w[name], y_out, rows, i, o, bias=b)
    e = mlk.DeviceBuffer.empty
    h, q, k, v, a, proj = e((T, D)), e((T, QD)), e((T, KD)), e((T, KD)), e((T, QD)), e((T, D))
    g, u = e((T, F)), e((T, F))
    mlk.rmsnorm(x2, an, h, T, D, cfg["eps"])
    linear("wq", h, q, T, D, QD, bias["wq"])
    linear("wk", h, k, T, D, KD, bias["wk"])
    linear("wv", h, v, T, D, KD, bias["wv"])
    mlk.rope(q, k, T, H, KV, hd, positions=positions, pos0=pos, theta=cfg["theta"],
             rope_type=cfg["rope_type"], err=flag2)
    mlk.kv_write(kc2, vc2, 1, S, KV, hd, 0, k, v, T, positions=positions, pos0=pos, err=flag2)
    nws = mlk.attention_workspace_bytes(T, H, KV, hd, S)
    aws = mlk.DeviceBuffer(max(nws, 16), np.uint8)
    mlk.attention_decode(q, kc2, vc2, 1, S, H, KV, hd, 0, T, a, S, positions=positions,
                         pos0=pos, workspace=aws, workspace_bytes=aws.nbytes, err=flag2)
    linear("wo", a, proj, T, QD, D)
    mlk.add_rmsnorm(x2, proj, fn, h, T, D, cfg["eps"])
    linear("w_gate", h, g, T, D, F)
    linear("w_up", h, u, T, D, F)
    mlk.swiglu(g, u, g, T * F)
    linear("w_down", g, proj, T, F, D)
    mlk.add(x2, proj, x2, T * D)
    want = x2.download()
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(kc.download(), kc2.download())
    np.testing.assert_array_equal(vc.download(), vc2.download())
    assert int(flag.download()[0]) == int(flag2.download()[0]) == (1 if case == "bad_position" else 0)
    if case == "bad_position":
        # the rows of the other positions were written, the cache outside them kept
        kept = np.setdiff1d(np.arange(S), pv)
        np.testing.assert_array_equal(kc.download()[0, kept], kc0[0, kept])


TILED_CASES = [  # dim, hidden, heads, tokens, wo/gate/up/down biases, RoPE layout
    (2048, 3072, 16, 4096, False, 0), (2048, 3072, 16, 4096, True, 0),
    (2048, 3072, 16, 4000, False, 0), (2048, 3072, 16, 4000, True, 0),
    (4096, 2048, 32, 4096, True, 0), (2048, 3072, 16, 4000, True, 1)]


@pytest.mark.parametrize("wt", ["q8_0", "q4_0"])
@pytest.mark.parametrize("D,F,H,T,biases,rope_type", TILED_CASES)
def test_layer_tiled_epilogues_equal_op_by_op(mlk, fwd, wt, D, F, H, T, biases, rope_type):
    """A prompt chunk large enough that wo, gate/up and down each take the
    128-row tile GEMM in one K pass (512 and more tiles of 128 outputs)
    carries their epilogues in that GEMM: wo and down add into the
    residual stream (then plain RMSNorm for the ffn input), gate and up run
    as one launch that writes SwiGLU(gate, up).  k and v (1024 outputs each)
    run as one launch without a K split, straight into their cache rows,
    where the RoPE launch rotates k (q in place; normal and NeoX layouts).
    The sums are the plain
    GEMM's (for k and v the unsplit one's: no workspace), so the layer
    equals the separate entry points bit for bit, with biases on all seven
    matrices too (T = 4000: a partial last tile, at positions 90..4089).  dim 2048 takes the
    residual adds on 128-output tiles, dim 4096 (Llama-3-8B's wo and down)
    on 256-output ones."""
    S, KV, hd = 4096, 8, 128
    p0 = 0 if T == 4096 else 90
    cfg = dict(vocab=64, dim=D, hidden_dim=F, layers=1, n_heads=H, n_kv_heads=KV,
               head_dim=hd, max_seq=S, rope_type=rope_type, theta=500000.0, eps=1e-5)
    model = O.forward_model(cfg, seed=17, weight_type=wt, biases=True)
    QD, KD = H * hd, KV * hd
    lw = model["layers"][0]
    dm = fwd.DeviceModel(model)
    rng = np.random.default_rng(9)
    B = mlk.DeviceBuffer.from_array
    extra = {}
    if biases:
        for n, o in (("wo", D), ("w_gate", F), ("w_up", F), ("w_down", D)):
            extra[n] = B((rng.standard_normal(o) * 0.1).astype(np.float32))
            getattr(dm.layers[0], n).bias = extra[n].ptr
    x0 = rng.standard_normal((T, D)).astype(np.float32)
    kc0 = np.zeros((1, S, KV, hd), np.float32)
    vc0 = np.zeros((1, S, KV, hd), np.float32)

    x, kc, vc = B(x0), B(kc0), B(vc0)
    ws = mlk.DeviceBuffer(fwd.layer_workspace_bytes(cfg, T, S, True), np.uint8)
    fwd.forward_layer_batch(cfg, dm.layers[0], x, T, kc, vc, 1, S, 0, S, ws, pos0=p0)
    got = x.download()

    w = {n: B(np.ascontiguousarray(lw[n][1], np.uint8)) for n in fwd.LINEAR_NAMES}
    bias = {n: B(np.asarray(lw["b" + n[1]], np.float32)) for n in ("wq", "wk", "wv")}
    bias.update(extra)
    an = B(np.asarray(lw["attention_norm"], np.float32))
    fn = B(np.asarray(lw["ffn_norm"], np.float32))
    x2, kc2, vc2 = B(x0), B(kc0), B(vc0)
    e = mlk.DeviceBuffer.empty
    h, q, k, v, a, proj = e((T, D)), e((T, QD)), e((T, KD)), e((T, KD)), e((T, QD)), e((T, D))
    g, u = e((T, F)), e((T, F))

    def linear(name, x_in, y_out, i, o, ws="auto"):
        mlk.linear_quant(wt, x_in, w[name], y_out, T, i, o, bias=bias.get(name), workspace=ws)
    mlk.rmsnorm(x2, an, h, T, D, cfg["eps"])
    linear("wq", h, q, D, QD)
    linear("wk", h, k, D, KD, ws=None)
    linear("wv", h, v, D, KD, ws=None)
    mlk.rope(q, k, T, H, KV, hd, pos0=p0, theta=cfg["theta"], rope_type=rope_type)
    mlk.kv_write(kc2, vc2, 1, S, KV, hd, 0, k, v, T, pos0=p0)
    nws = mlk.attention_workspace_bytes(T, H, KV, hd, S)
    aws = mlk.DeviceBuffer(max(nws, 16), np.uint8)
    mlk.attention_decode(q, kc2, vc2, 1, S, H, KV, hd, 0, T, a, S, pos0=p0, workspace=aws,
                         workspace_bytes=aws.nbytes)
    linear("wo", a, proj, QD, D)
    mlk.add_rmsnorm(x2, proj, fn, h, T, D, cfg["eps"])
    linear("w_gate", h, g, D, F)
    linear("w_up", h, u, D, F)
    mlk.swiglu(g, u, g, T * F)
    linear("w_down", g, proj, F, D)
    mlk.add(x2, proj, x2, T * D)
    np.testing.assert_array_equal(got, x2.download())
    np.testing.assert_array_equal(kc.download(), kc2.download())
    np.testing.assert_array_equal(vc.download(), vc2.download())


@pytest.mark.parametrize("wt", ["q8_0", "q4_0"])
@pytest.mark.parametrize("D,F", [(2048, 1024), (4096, 1024), (6144, 512), (8192, 512)])
@pytest.mark.parametrize("planar", [False, True])
def test_one_token_norms_folded_equal_op_by_op(mlk, fwd, wt, D, F, planar):
    """One token with dim 2048..8192: both RMSNorms are staged inside the
    streaming q/k/v and gate/up launches (the norm kernel's block of 8 or 16
    waves with one or two float4s per thread, the second partly used at
    6144, emulated there: its float64 sums in the same order), and the
    residual x + proj reaches the down projection through the h buffer.  The
    layer equals the separate entry points bit for bit, over the blocks and
    over planar copies (then each matrix through mlk_linear_planar)."""
    S, H, KV, hd, pos = 256, 16, 4, 128, 200
    cfg = dict(vocab=64, dim=D, hidden_dim=F, layers=1, n_heads=H, n_kv_heads=KV,
               head_dim=hd, max_seq=S, rope_type=0, theta=500000.0, eps=1e-5)
    model = O.forward_model(cfg, seed=D + F, weight_type=wt, biases=False)
    QD, KD = H * hd, KV * hd
    lw = model["layers"][0]
    dm = fwd.DeviceModel(model, planar=planar)
    rng = np.random.default_rng(D)
    x0 = (rng.standard_normal((1, D)) * 3).astype(np.float32)
    kc0 = (rng.standard_normal((1, S, KV, hd)) * 0.5).astype(np.float32)
    vc0 = rng.standard_normal((1, S, KV, hd)).astype(np.float32)
    B = mlk.DeviceBuffer.from_array
    x, kc, vc = B(x0), B(kc0), B(vc0)
    ws = mlk.DeviceBuffer(fwd.layer_workspace_bytes(cfg, 1, S, True), np.uint8)
    fwd.forward_layer_batch(cfg, dm.layers[0], x, 1, kc, vc, 1, S, 0, S, ws, pos0=pos)
    got = x.download()

    def up(a):
        return B(np.ascontiguousarray(a))
    w = {n: up(np.asarray(lw[n][1], np.uint8)) for n in fwd.LINEAR_NAMES}
    shapes = {"wq": (QD, D), "wk": (KD, D), "wv": (KD, D), "wo": (D, QD), "w_gate": (F, D),
              "w_up": (F, D), "w_down": (D, F)}
    if planar:
        for n, (o, i) in shapes.items():
            pw = mlk.DeviceBuffer(mlk.quant_planar_bytes(wt, o, i), np.uint8)
            mlk.quant_to_planar(wt, w[n], o, i, pw)
            w[n] = pw

    def linear(name, x_in, y_out):
        o, i = shapes[name]
        if planar:
            mlk.linear_planar(wt, x_in, w[name], y_out, 1, i, o, workspace=None)
        else:
            mlk.linear_quant(wt, x_in, w[name], y_out, 1, i, o)
    an, fn = up(np.asarray(lw["attention_norm"], np.float32)), up(np.asarray(lw["ffn_norm"], np.float32))
    x2, kc2, vc2 = B(x0), B(kc0), B(vc0)
    e = mlk.DeviceBuffer.empty
    h, q, k, v, a, proj = e((1, D)), e((1, QD)), e((1, KD)), e((1, KD)), e((1, QD)), e((1, D))
    g, u = e((1, F)), e((1, F))
    mlk.rmsnorm(x2, an, h, 1, D, cfg["eps"])
    linear("wq", h, q)
    linear("wk", h, k)
    linear("wv", h, v)
    mlk.rope(q, k, 1, H, KV, hd, pos0=pos, theta=cfg["theta"], rope_type=0)
    mlk.kv_write(kc2, vc2, 1, S, KV, hd, 0, k, v, 1, pos0=pos)
    nws = mlk.attention_workspace_bytes(1, H, KV, hd, S)
    aws = mlk.DeviceBuffer(max(nws, 16), np.uint8)
    mlk.attention_decode(q, kc2, vc2, 1, S, H, KV, hd, 0, 1, a, S, pos0=pos, workspace=aws,
                         workspace_bytes=aws.nbytes)
    linear("wo", a, proj)
    mlk.add_rmsnorm(x2, proj, fn, h, 1, D, cfg["eps"])
    linear("w_gate", h, g)
    linear("w_up", h, u)
    mlk.swiglu(g, u, g, F)
    linear("w_down", g, proj)
    mlk.add(x2, proj, x2, D)
    np.testing.assert_array_equal(got, x2.download())
    np.testing.assert_array_equal(kc.download(), kc2.download())
    np.testing.assert_array_equal(vc.download(), vc2.download())


@pytest.mark.parametrize("wt", ["q8_0", "q4_0"])
@pytest.mark.parametrize("T", [1, 2, 12, 24])
@pytest.mark.parametrize("case", ["pos0", "positions", "bad_position", "neox"])
def test_layer_planar_equals_op_by_op(mlk, fwd, wt, T, case):
    """With planar copies of the weights, 1..32 tokens take the planar
    launches: q/k/v in one (RoPE and the K/V cache rows in its epilogue or
    reduction for the normal layout; one token also stages the RMSNorm),
    gate/up with SwiGLU, down adding into x, and wo.
    Their per-element arithmetic is the separate entries' (mlk_linear_planar
    per matrix, then the separate ops), so the layer equals that composition
    bit for bit: residual stream, cache rows and error flag."""
    cfg = dict(vocab=64, dim=512, hidden_dim=1536, layers=1, n_heads=8, n_kv_heads=2,
               head_dim=64, max_seq=1024, rope_type=1 if case == "neox" else 0, theta=10000.0,
               eps=1e-5)
    layer_planar_vs_op_by_op(mlk, fwd, wt, T, case, cfg)


@pytest.mark.parametrize("wt", ["q8_0", "q4_0"])
def test_layer_planar_equals_op_by_op_70b(mlk, fwd, wt):
    """The same at Llama-3-70B's layer shape with 16 tokens, where the fused
    launches take the streaming planar GEMM (more row groups than the
    one-shot grid spreads well): q/k/v as three segments of one launch (RoPE
    and the cache rows in its reduction), gate/up as two (SwiGLU), down with
    its split-K partials (the residual add).  Separately, q, k and v each
    take the one-shot kernel and gate, up and down the streaming one on a
    single segment.  Equal bit for bit."""
    cfg = dict(vocab=64, dim=8192, hidden_dim=28672, layers=1, n_heads=64, n_kv_heads=8,
               head_dim=128, max_seq=1024, rope_type=0, theta=500000.0, eps=1e-5)
    layer_planar_vs_op_by_op(mlk, fwd, wt, 16, "pos0", cfg)


def layer_planar_vs_op_by_op(mlk, fwd, wt, T, case, cfg):
    """One layer through forward_layer_batch on planar copies against the
    separate entries on the same blocks (see the tests above)."""
    S = cfg["max_seq"]
    model = O.forward_model(cfg, seed=13, weight_type=wt, biases=True)
    D, F, H, KV, hd = (cfg[k] for k in ("dim", "hidden_dim", "n_heads", "n_kv_heads", "head_dim"))
    QD, KD, pos = H * hd, KV * hd, 600
    lw = model["layers"][0]
    dm = fwd.DeviceModel(model, planar=True)
    rng = np.random.default_rng(7)
    x0 = rng.standard_normal((T, D)).astype(np.float32)
    kc0 = (rng.standard_normal((1, S, KV, hd)) * 0.5).astype(np.float32)
    vc0 = rng.standard_normal((1, S, KV, hd)).astype(np.float32)
    B = mlk.DeviceBuffer.from_array
    positions = None
    if case in ("positions", "bad_position"):
        pv = np.sort(rng.choice(S, T, replace=False)).astype(np.int32)
        if case == "bad_position":
            pv[T // 2] = S
        positions = B(pv)
    contiguous = positions is None
    flag, flag2 = B(np.zeros(1, np.int32)), B(np.zeros(1, np.int32))

    x = B(x0)
    kc, vc = B(kc0), B(vc0)
    ws = mlk.DeviceBuffer(fwd.layer_workspace_bytes(cfg, T, S, contiguous), np.uint8)
    fwd.forward_layer_batch(cfg, dm.layers[0], x, T, kc, vc, 1, S, 0, S, ws, positions=positions,
                            pos0=pos, err=flag)
    got = x.download()

    shapes = {"wq": (QD, D), "wk": (KD, D), "wv": (KD, D), "wo": (D, QD), "w_gate": (F, D),
              "w_up": (F, D), "w_down": (D, F)}
    pw = {}
    for n, (o, i) in shapes.items():
        blocks = B(np.ascontiguousarray(lw[n][1], np.uint8))
        pw[n] = mlk.DeviceBuffer(mlk.quant_planar_bytes(wt, o, i), np.uint8)
        mlk.quant_to_planar(wt, blocks, o, i, pw[n])
    bias = {n: B(np.asarray(lw["b" + n[1]], np.float32)) for n in ("wq", "wk", "wv")}
    an = B(np.asarray(lw["attention_norm"], np.float32))
    fn = B(np.asarray(lw["ffn_norm"], np.float32))
    x2, kc2, vc2 = B(x0), B(kc0), B(vc0)
    e = mlk.DeviceBuffer.empty
    h, q, k, v, a, proj = e((T, D)), e((T, QD)), e((T, KD)), e((T, KD)), e((T, QD)), e((T, D))
    g, u = e((T, F)), e((T, F))
    mlk.rmsnorm(x2, an, h, T, D, cfg["eps"])
    mlk.linear_planar(wt, h, pw["wq"], q, T, D, QD, bias=bias["wq"])
    mlk.linear_planar(wt, h, pw["wk"], k, T, D, KD, bias=bias["wk"])
    mlk.linear_planar(wt, h, pw["wv"], v, T, D, KD, bias=bias["wv"])
    mlk.rope(q, k, T, H, KV, hd, positions=positions, pos0=pos, theta=cfg["theta"],
             rope_type=cfg["rope_type"], err=flag2)
    mlk.kv_write(kc2, vc2, 1, S, KV, hd, 0, k, v, T, positions=positions, pos0=pos, err=flag2)
    nws = mlk.attention_workspace_bytes(T, H, KV, hd, S)
    aws = mlk.DeviceBuffer(max(nws, 16), np.uint8)
    mlk.attention_decode(q, kc2, vc2, 1, S, H, KV, hd, 0, T, a, S, positions=positions,
                         pos0=pos, workspace=aws, workspace_bytes=aws.nbytes, err=flag2)
    mlk.linear_planar(wt, a, pw["wo"], proj, T, QD, D)
    mlk.add_rmsnorm(x2, proj, fn, h, T, D, cfg["eps"])
    mlk.linear_planar(wt, h, pw["w_gate"], g, T, D, F)
    mlk.linear_planar(wt, h, pw["w_up"], u, T, D, F)
    mlk.swiglu(g, u, g, T * F)
    mlk.linear_planar(wt, g, pw["w_down"], proj, T, F, D)
    mlk.add(x2, proj, x2, T * D)
    np.testing.assert_array_equal(got, x2.download())
    np.testing.assert_array_equal(kc.download(), kc2.download())
    np.testing.assert_array_equal(vc.download(), vc2.download())
    assert int(flag.download()[0]) == int(flag2.download()[0]) == (1 if case == "bad_position" else 0)


@pytest.mark.parametrize("wt", ["q8_0", "q4_0"])
def test_forward_planar_matches_oracle(orc, fwd, wt):
    """A model with planar copies: decode steps of 1 token and batches of 2,
    5, 16 and 32 tokens (the planar kernels) after a 33-token prefill (the
    GEMM on the blocks),
    against the reference's ForwardToken loop over the same tokens."""
    cfg = dict(vocab=300, dim=512, hidden_dim=1024, layers=2, n_heads=8, n_kv_heads=2,
               head_dim=64, max_seq=160, rope_type=0, theta=10000.0, eps=1e-5)
    model = O.forward_model(cfg, seed=21, weight_type=wt, biases=True)
    sizes = [33, 1, 2, 5, 1, 16, 32]
    n = sum(sizes)
    rng = np.random.default_rng(4)
    tokens = rng.integers(0, cfg["vocab"], n).astype(np.int32)
    want, _ = orc.forward_tokens(model, tokens, np.arange(n, dtype=np.int32))
    dm = fwd.DeviceModel(model, planar=True)
    at = 0
    for T in sizes:
        got = dm.forward(tokens[at:at + T], pos0=at, all_logits=True)
        assert_forward_close(got, want[at:at + T], f"{wt} batch of {T} at {at}")
        at += T


LAYER_8B = dict(dim=4096, hidden_dim=14336, n_heads=32, n_kv_heads=8, head_dim=128, layers=1,
                rope_type=0, theta=500000.0, eps=1e-5)
S_8B = 8192


def host_layer_8b(orc, qt, seed):
    """One Llama-3-8B-shaped layer on the host: norm weights N(1, 0.1),
    projections N(0, 0.02) quantized by the oracle (the reference's
    quantizer, bit for bit)."""
    c = LAYER_8B
    D, F = c["dim"], c["hidden_dim"]
    QD, KD = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    rng = np.random.default_rng(seed)
    lw = {"attention_norm": (1 + 0.1 * rng.standard_normal(D)).astype(np.float32),
          "ffn_norm": (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)}
    for name, (o, i) in {"wq": (QD, D), "wk": (KD, D), "wv": (KD, D), "wo": (D, QD),
                         "w_gate": (F, D), "w_up": (F, D), "w_down": (D, F)}.items():
        w = (0.02 * rng.standard_normal((o, i), dtype=np.float32))
        lw[name] = (qt, orc.quantize(qt, w))
        lw[name + "_shape"] = (o, i)
    return lw


def gamma(n):
    return n * U32 / (1 - n * U32)


@pytest.mark.parametrize("qt", ["q8_0", "q4_0"])
def test_layer_8b_decode_planar_matches_oracle(mlk, orc, fwd, qt):
    """The decode steps the bench times, at the Llama-3-8B layer shape on
    planar Q8_0 / Q4_0 weights (the path of 1..32 tokens) over a cache
    pre-filled at every position 0..8191: one token at position 8191
    (streaming GEMVs, attention over 8192 rows), and 16 tokens at distinct
    positions uniform in 0..8191 (planar matrix-core linears, shared-tile
    attention).  Against the oracle's op-by-op composition of the same step
    (ForwardBatch's token loop over one layer, src/forward.cc:482-486 and
    ForwardLayer :385-414) with the same weights and cache.

    The bars.  The reference's forward bar 1e-5 + 1e-4|x| was set on its
    tiny model (dim 32); at this shape the last op sums 14336 fp32 terms of
    size ~1e-2, and an fp32 sum in any order is only within
    gamma_K * sum|terms| of the exact one: measured here, both the oracle's
    serial sum and the device's split sums land up to ~2-3e-5 from the exact
    value near x = 0, beyond 1e-5.  So the forward bar gets the summation
    bound of the down projection added (f = the oracle's SwiGLU output,
    S_j = sum_k |f_k w_jk|):
      - the layer output against the oracle's own fp32 result: the forward
        bar + 2 gamma_F S (both sums);
      - the layer output against r + f W_down^T evaluated in float64 over
        the oracle's own residual r and f: the forward bar + gamma_F S (the
        device's sum alone);
      - the K / V rows each token wrote against the oracle's: 1e-5 + 1e-4|k|
        plus 2 gamma_D sum_i |h_i w_ji| (over both rows of a rotated pair
        for K).
    Each case prints its largest error as a multiple of the plain forward
    bar."""
    c = LAYER_8B
    D, F, KV, hd = c["dim"], c["hidden_dim"], c["n_kv_heads"], c["head_dim"]
    lw = host_layer_8b(orc, qt, seed=17 if qt == "q8_0" else 18)
    keep = []

    def up(a):
        buf = mlk.DeviceBuffer.from_array(np.ascontiguousarray(a))
        keep.append(buf)
        return buf

    w = fwd.LayerWeights()
    w.attention_norm = up(lw["attention_norm"]).ptr
    w.ffn_norm = up(lw["ffn_norm"]).ptr
    for name in fwd.LINEAR_NAMES:
        o, i = lw[name + "_shape"]
        blocks = up(lw[name][1])
        pl = mlk.DeviceBuffer(mlk.quant_planar_bytes(qt, o, i), np.uint8)
        mlk.quant_to_planar(qt, blocks, o, i, pl)
        keep.append(pl)
        lin = fwd.LinearWeight()
        lin.type, lin.data, lin.bias, lin.planar = mlk.QUANT[qt], blocks.ptr, None, pl.ptr
        setattr(w, name, lin)
    wd = orc.dequantize(qt, lw["w_down"][1], D, F).astype(np.float64)
    wk = np.abs(orc.dequantize(qt, lw["wk"][1], KV * hd, D).astype(np.float64))
    wv = np.abs(orc.dequantize(qt, lw["wv"][1], KV * hd, D).astype(np.float64))
    rng = np.random.default_rng(5)
    kc0 = rng.standard_normal((1, S_8B, KV, hd), dtype=np.float32)
    vc0 = rng.standard_normal((1, S_8B, KV, hd), dtype=np.float32)
    spos = np.sort(rng.choice(S_8B, 16, replace=False)).astype(np.int32)
    for T, positions in ((1, np.array([S_8B - 1], np.int32)), (16, spos)):
        print(f"8B layer {qt}: T={T} positions {positions[:4]}...{positions[-1]}", flush=True)
        x = rng.standard_normal((T, D), dtype=np.float32)
        kc, vc = kc0.copy(), vc0.copy()
        inter = []
        want = orc.layer_tokens(c, lw, x, kc, vc, 0, positions, keep=inter).astype(np.float64)
        f = np.stack([d["f"] for d in inter]).astype(np.float64)
        r = np.stack([d["r"] for d in inter]).astype(np.float64)
        h = np.abs(np.stack([d["h"] for d in inter]).astype(np.float64))
        d_x, d_k, d_v = up(x), up(kc0), up(vc0)
        consecutive = T == 1
        max_ctx = int(positions.max()) + 1
        ws = mlk.DeviceBuffer(fwd.layer_workspace_bytes(c, T, max_ctx, consecutive), np.uint8)
        d_pos = None if consecutive else up(positions)
        fwd.forward_layer_batch(c, w, d_x, T, d_k, d_v, 1, S_8B, 0, max_ctx, ws,
                                positions=d_pos, pos0=int(positions[0]))
        mlk.synchronize()
        got = d_x.download().astype(np.float64)
        assert np.isfinite(got).all()
        err = np.abs(got - want)
        bar = 1e-5 + 1e-4 * np.abs(want)
        sum_bound = gamma(F) * (np.abs(f) @ np.abs(wd).T)
        assert (err <= bar + 2 * sum_bound).all(), (
            f"{qt} T={T}: {int((err > bar + 2 * sum_bound).sum())} outputs beyond the forward "
            "bar + both sums' bound")
        exact = r + f @ wd.T
        err64 = np.abs(got - exact)
        bar64 = 1e-5 + 1e-4 * np.abs(exact)
        assert (err64 <= bar64 + sum_bound).all(), (
            f"{qt} T={T}: {int((err64 > bar64 + sum_bound).sum())} outputs beyond the forward "
            "bar + the device sum's bound, against float64")
        print(f"8B layer {qt} T={T}: vs the oracle max |err| {float(err.max()):.2e} "
              f"({float((err / bar).max()):.2f} x the plain forward bar, "
              f"{int((err > bar).sum())} beyond it); vs the float64 down projection "
              f"{float(err64.max()):.2e} ({float((err64 / bar64).max()):.2f} x, "
              f"{int((err64 > bar64).sum())} beyond it); of {err.size}")
        s_k = h @ wk.T  # [T, KV*hd]
        s_k = s_k + s_k.reshape(T, -1, 2)[:, :, ::-1].reshape(T, -1)  # both rows of a pair
        s_v = h @ wv.T
        for cache_d, cache_h, s, what in ((d_k, kc, s_k, "K"), (d_v, vc, s_v, "V")):
            g_rows = cache_d.download()[0, positions].reshape(T, -1).astype(np.float64)
            w_rows = cache_h[0, positions].reshape(T, -1).astype(np.float64)
            e = np.abs(g_rows - w_rows)
            lim = 1e-5 + 1e-4 * np.abs(w_rows) + 2 * gamma(D) * s
            assert (e <= lim).all(), f"{qt} T={T} {what} rows: {int((e > lim).sum())} beyond"
