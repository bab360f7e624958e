"""Writes the golden fixtures in tests/golden/ from the compiled reference.

Runs only where the reference tree exists (oracle/_ref/libref.so is built
from the reference's own CPU sources by `make -C oracle ref`).  Every fixture
holds the inputs and the outputs the reference computed for them; the
reference itself never travels.  Re-run with:

    make -C oracle && python tests/golden/make_golden.py

Fixture contents (numpy .npz, no pickles):
  tiny_chain.npz   config 1 of BASELINE.json: gather -> residual add +
                   RmsNorm -> RoPE(q, k) -> SwiGLU on the 6-token prompt.
  quant.npz        TensorToQ80/Q40/Q41 blocks and Q*ToTensor rows for
                   N(0, 0.02) rows (dim 4096, the C4 table distribution),
                   ragged widths with tail blocks, and hand-made edge rows.
  dequant_kat.npz  hand-made blocks (scales 0, subnormal 0x0001, 0x3400,
                   0x3A00, 0x4000; Q4_1 minima -2, -0.5, 0, 1.5) and the
                   reference's dequantized values.
  rows_8b_70b.npz  RmsNorm / SwiGLU / Silu rows at the 8B and 70B widths,
                   RoPE heads at positions 0, 1, 4095, 8191 (theta 5e5) for
                   both layouts, softmax rows.
  linear.npz       LinearQ80/Q40/Q41 (default build) on the weight and input
                   patterns of the reference's own tests
                   (test/cuda_quant_test.cc:33-39 at [131, in] for in in
                   1, 17, 32, 33, 65; tests/cuda_test_support.h:43-47 at
                   [7, 32] and [7, 86]) and on N(0, 0.02) Llama-3-8B-width
                   rows; F32 Linear and Matmul on the shapes of
                   tests/test_cuda_linear.cc and tests/test_cuda_matmul.cc.
  attention.npz    decode attention for one query token (the reference's
                   own KvCache and ForwardAttention) on
                   the cases of test/cuda_attention_test.cc:86-88 (their
                   sin / cos inputs) and on an N(0, 1) GQA case with
                   head_dim 128 (8 query heads over 2 KV heads, pos 63).
  tiny_forward.npz the reference's tiny model (model/tinymodel, its float32
                   weights as the model file holds them) and the logits of
                   its own CPU forward pass (the ForwardToken loop of
                   ForwardBatch) for a 9-token prompt at positions 0..8.

Usage: make_golden.py [name ...] writes only the named fixtures.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as O  # noqa: E402


def normal(rng, shape, mean=0.0, std=1.0):
    return (rng.standard_normal(shape) * std + mean).astype(np.float32)


def tiny_chain(ref):
    """BASELINE.json configs[0]."""
    rng = np.random.default_rng(42)
    vocab, dim, H, KV, hd, F = 131, 64, 4, 2, 16, 172
    eps, theta = 1e-5, 10000.0
    ids = np.array([128, 104, 101, 108, 108, 111], dtype=np.int32)
    pos = np.arange(6, dtype=np.int32)
    T = len(ids)
    table = normal(rng, (vocab, dim), std=0.02)
    norm_w = normal(rng, (dim,), mean=1.0, std=0.1)
    q = normal(rng, (T, H * hd))
    k = normal(rng, (T, KV * hd))
    v = normal(rng, (T, KV * hd))  # drawn to keep the config's draw order; unused
    gate = normal(rng, (T, F))
    up = normal(rng, (T, F))
    # The residual branch is not given by the config: it is the next draw,
    # N(0, 0.02) like the embedding it is added to.
    delta = normal(rng, (T, dim), std=0.02)
    gathered = table[ids].copy()
    x = np.empty((T, dim), np.float32)
    y = np.empty((T, dim), np.float32)
    q_out = q.copy()
    k_out = k.copy()
    ffn = np.empty((T, F), np.float32)
    bufs = dict(table=table, vocab=vocab, dim=dim, ids=ids, x=x, delta=delta, norm_w=norm_w,
                y=y, eps=eps, q=q_out, k=k_out, n_heads=H, n_kv_heads=KV, head_dim=hd,
                positions=pos, theta=theta, gate=gate, up=up, ffn_out=ffn, ffn_dim=F)
    assert ref.chain(bufs, T, 1) == 0
    return dict(vocab=vocab, dim=dim, n_heads=H, n_kv_heads=KV, head_dim=hd, ffn_dim=F,
                eps=np.float32(eps), theta=np.float32(theta), ids=ids, positions=pos,
                table=table, norm_w=norm_w, q=q, k=k, v=v, gate=gate, up=up, delta=delta,
                gathered=gathered, residual_out=x, norm_out=y, q_out=q_out, k_out=k_out,
                ffn_out=ffn)


def edge_rows():
    """Rows that exercise quantizer corner cases."""
    rows = np.zeros((6, 64), np.float32)
    rows[1] = 0.5                                        # constant row
    rows[2, :32] = np.linspace(-1, 1, 32)                # signed ramp
    rows[2, 32:] = np.linspace(3, -7, 32)
    rows[3, ::2] = 1e-6                                  # tiny values (subnormal fp16 scale)
    rows[3, 1::2] = -3e-7
    rows[4, :] = 127.0 * np.arange(-32, 32) / 64.0       # exact .5 ties for Q8_0
    rows[5, :] = 65504.0 * np.sign(np.arange(64) - 31.5)  # fp16 overflow boundary
    return rows


def quant(ref):
    rng = np.random.default_rng(7)
    out = {}
    cases = {
        "c4": normal(rng, (4, 4096), std=0.02),
        "ragged100": normal(rng, (3, 100), std=1.0),
        "ragged33": normal(rng, (2, 33), std=0.5),
        "ragged7": normal(rng, (2, 7), std=2.0),
        "edge": edge_rows(),
    }
    for name, x in cases.items():
        out[f"{name}_x"] = x
        for qt in O.QUANT_TYPES:
            blocks = ref.quantize(qt, x)
            out[f"{name}_{qt}_blocks"] = blocks
            out[f"{name}_{qt}_deq"] = ref.dequantize(qt, blocks, x.shape[0], x.shape[1])
    return out


def dequant_kat(ref):
    """Hand-made blocks in the style of the reference's handcrafted tests."""
    scales = [0x0000, 0x0001, 0x3400, 0x3A00, 0x4000]
    minima = [0xC000, 0xB800, 0x0000, 0x3E00]
    rows, nb = 5, 4
    cols = nb * 32
    q8 = np.zeros((rows, nb, 34), np.uint8)
    q40 = np.zeros((rows, nb, 18), np.uint8)
    q41 = np.zeros((rows, nb, 20), np.uint8)
    for r in range(rows):
        for b in range(nb):
            d = scales[(r + b) % 5]
            q8[r, b, 0:2] = [d & 0xFF, d >> 8]
            q40[r, b, 0:2] = [d & 0xFF, d >> 8]
            d41 = scales[(r + b) % 5]
            m = minima[(r + b) % 4]
            q41[r, b, 0:4] = [d41 & 0xFF, d41 >> 8, m & 0xFF, m >> 8]
            for i in range(32):
                q8[r, b, 2 + i] = (i * 37 + r * 19 + b * 13) % 256
            for i in range(16):
                lo = (i * 3 + r + b) % 16
                hi = (i * 5 + r * 7 + b + 3) % 16
                q40[r, b, 2 + i] = lo | (hi << 4)
                q41[r, b, 4 + i] = lo | (hi << 4)
    out = {"rows": rows, "cols": cols}
    for qt, blk in (("q8_0", q8), ("q4_0", q40), ("q4_1", q41)):
        flat = blk.reshape(-1).copy()
        out[f"{qt}_blocks"] = flat
        out[f"{qt}_deq"] = ref.dequantize(qt, flat, rows, cols)
        out[f"{qt}_deq_flat"] = ref.dequantize(qt, flat, rows, cols, flat=True)
    return out


def rows_8b_70b(ref):
    rng = np.random.default_rng(11)
    out = {}
    for tag, dim, ffn in (("8b", 4096, 14336), ("70b", 8192, 28672)):
        x = normal(rng, (dim,), std=0.02)
        w = normal(rng, (dim,), mean=1.0, std=0.1)
        out[f"rms_{tag}_x"], out[f"rms_{tag}_w"] = x, w
        out[f"rms_{tag}_y"] = ref.rmsnorm_row(x, w, 1e-5)
        g = normal(rng, (ffn,), std=0.02)
        u = normal(rng, (ffn,), std=0.02)
        out[f"swiglu_{tag}_g"], out[f"swiglu_{tag}_u"] = g, u
        out[f"swiglu_{tag}_y"] = ref.swiglu(g, u)
        # unit-scale gate for a wide SiLU argument range
        g1 = normal(rng, (4096,), std=4.0)
        out[f"silu_{tag}_x"] = g1
        out[f"silu_{tag}_y"] = ref.silu(g1)
    H, KV, hd, theta = 32, 8, 128, 500000.0
    for pos in (0, 1, 4095, 8191):
        q = normal(rng, (H * hd,), std=0.02)
        k = normal(rng, (KV * hd,), std=0.02)
        out[f"rope_p{pos}_q"], out[f"rope_p{pos}_k"] = q, k
        for rt, name in ((O.ROPE_NORMAL, "normal"), (O.ROPE_NEOX, "neox")):
            qo, ko = ref.rope_token(q, k, H, KV, hd, pos, theta, rt)
            out[f"rope_p{pos}_{name}_q"], out[f"rope_p{pos}_{name}_k"] = qo, ko
    sm = normal(rng, (1025,), std=3.0)
    out["softmax_x"] = sm
    out["softmax_y"] = ref.softmax(sm)
    big = np.array([-1000, 0, 1000, 999, -999], np.float32)
    out["softmax_big_x"] = big
    out["softmax_big_y"] = ref.softmax(big)
    return out


def pattern_43(shape):
    """test/cuda_quant_test.cc:33-39: ((i * 17 + 3) % 43 - 21) / 16."""
    i = np.arange(int(np.prod(shape)), dtype=np.int64)
    return (((i * 17 + 3) % 43 - 21).astype(np.float32) / np.float32(16)).reshape(shape)


def pattern_sin(shape, phase=0.0):
    """tests/cuda_test_support.h:43-47: sin(float(i) * 0.19f + phase) * 0.3f,
    evaluated in float32 like the C++ expression, then sin in float64 and
    rounded (std::sin of a float argument)."""
    i = np.arange(int(np.prod(shape)), dtype=np.float32)
    arg = i * np.float32(0.19) + np.float32(phase)
    return (np.sin(arg.astype(np.float64)).astype(np.float32) * np.float32(0.3)).reshape(shape)


def linear(ref):
    out = {}
    qts = ("q8_0", "q4_0", "q4_1")
    for qt in qts:
        for inf in (1, 17, 32, 33, 65):
            w = pattern_43((131, inf))
            blocks = ref.quantize(qt, w)
            out[f"p43_{qt}_{inf}_w"] = blocks
            for rows in (1, 3):
                x = pattern_43((rows, inf))
                out[f"p43_{qt}_{inf}_x{rows}"] = x
                out[f"p43_{qt}_{inf}_y{rows}"] = ref.linear_quant(qt, x, blocks, 131)
        for cols in (32, 86):
            w = pattern_sin((7, cols), 0.8)
            blocks = ref.quantize(qt, w)
            x = pattern_sin((1, cols))
            out[f"sin_{qt}_{cols}_w"] = blocks
            out[f"sin_{qt}_{cols}_x"] = x
            out[f"sin_{qt}_{cols}_y"] = ref.linear_quant(qt, x, blocks, 7)
        rng = np.random.default_rng(5)
        for out_f, inf, rows in ((32, 4096, 3), (8, 14336, 2)):
            w = normal(rng, (out_f, inf), std=0.02)
            blocks = ref.quantize(qt, w)
            x = normal(rng, (rows, inf), std=1.0)
            tag = f"n_{qt}_{out_f}x{inf}"
            out[f"{tag}_w"], out[f"{tag}_x"] = blocks, x
            out[f"{tag}_y"] = ref.linear_quant(qt, x, blocks, out_f)
    out["sin_bias7"] = pattern_sin((7,), 0.4)
    w = pattern_sin((17, 33), 0.3)
    out["f32_w"] = w
    out["f32_bias"] = pattern_sin((17,), 0.2)
    out["f32_x"] = pattern_sin((1, 33))
    out["f32_y"] = ref.linear_f32(out["f32_x"], w)
    for m, k, n in ((3, 7, 5), (1, 33, 17)):
        a, b = pattern_sin((m, k)), pattern_sin((k, n), 0.7)
        out[f"mm_{m}x{k}x{n}_a"], out[f"mm_{m}x{k}x{n}_b"] = a, b
        out[f"mm_{m}x{k}x{n}_c"] = ref.matmul_f32(a, b)
    return out


def attention(ref):
    out = {}
    cases = (("c0", 2, 2, 7, 0, 0), ("c1", 4, 2, 9, 5, 1), ("c2", 4, 1, 133, 130, 1))
    for name, H, KV, hd, pos, layer in cases:
        # test/cuda_attention_test.cc:90-103: cache of 2 layers, pos + 2 slots
        S = pos + 2
        q = np.sin(np.arange(H * hd, dtype=np.float32) * np.float32(0.17)).reshape(H, hd)
        i = np.arange(KV * hd, dtype=np.float32)
        k = np.stack([np.cos(i * np.float32(0.13) + np.float32(t * 0.1)) for t in range(S)])
        v = np.stack([np.sin(i * np.float32(0.11) - np.float32(t * 0.2)) for t in range(S)])
        k = k.astype(np.float32).reshape(S, KV, hd)
        v = v.astype(np.float32).reshape(S, KV, hd)
        out[f"{name}_q"], out[f"{name}_k"], out[f"{name}_v"] = q.astype(np.float32), k, v
        out[f"{name}_shape"] = np.array([H, KV, hd, pos, layer, 2, S], np.int32)
        out[f"{name}_out"] = ref.attention(q, k[:pos + 1], v[:pos + 1], 2, S, layer, pos)
    rng = np.random.default_rng(21)
    H, KV, hd, pos = 8, 2, 128, 63
    q = normal(rng, (H, hd))
    k, v = normal(rng, (pos + 1, KV, hd)), normal(rng, (pos + 1, KV, hd))
    out["g_q"], out["g_k"], out["g_v"] = q, k, v
    out["g_shape"] = np.array([H, KV, hd, pos, 0, 1, pos + 1], np.int32)
    out["g_out"] = ref.attention(q, k, v, 1, pos + 1, 0, pos)
    return out


REF_ROOT = os.environ.get("MINILAMMA_REFERENCE", "/root/reference")  # the reference tree
TINY_DIR = os.path.join(REF_ROOT, "model", "tinymodel")
TINY_TOKENS = [128, 104, 101, 108, 108, 111, 32, 119, 111]  # BOS "hello wo"


def tiny_model():
    """The reference's tiny model (model/tinymodel: model.json lists the
    tensors, model.bin holds them as raw little-endian float32) in
    oracle.forward_model layout."""
    import json
    with open(os.path.join(TINY_DIR, "model.json")) as f:
        meta = json.load(f)
    raw = np.fromfile(os.path.join(TINY_DIR, "model.bin"), dtype="<f4")
    t = {e["name"]: raw[e["offset"] // 4:(e["offset"] + e["byte_size"]) // 4].reshape(e["shape"])
         for e in meta["tensors"]}
    c = meta["config"]
    config = dict(vocab=c["vocab_size"], dim=c["dim"], hidden_dim=c["hidden_dim"],
                  layers=c["layers"], n_heads=c["n_heads"], n_kv_heads=c["n_kv_heads"],
                  head_dim=c["head_dim"], max_seq=c["max_seq_len"], rope_type=0,
                  theta=c["rope_theta"], eps=c["rms_norm_eps"])
    layers = []
    for i in range(config["layers"]):
        p = f"layers.{i}."
        lw = {n: t[p + n].astype(np.float32) for n in ("attention_norm", "ffn_norm")}
        for n in O.LINEAR_NAMES:
            lw[n] = ("f32", t[p + n].astype(np.float32))
        layers.append(lw)
    return {"config": config, "embedding": t["token_embedding"].astype(np.float32),
            "layers": layers, "final_norm": t["final_norm"].astype(np.float32),
            "lm_head": ("f32", t["lm_head"].astype(np.float32))}


def tiny_forward(ref):
    """The reference's ForwardToken loop (its own CPU forward pass) on its
    tiny model, for a 9-token prompt at positions 0..8: the weights (as the
    model file holds them), the config and every step's logits."""
    m = tiny_model()
    out = {"config": np.array([m["config"][k] for k in ("vocab", "dim", "hidden_dim", "layers",
                                                       "n_heads", "n_kv_heads", "head_dim",
                                                       "max_seq", "rope_type")], np.int32),
           "theta_eps": np.array([m["config"]["theta"], m["config"]["eps"]], np.float32),
           "embedding": m["embedding"], "final_norm": m["final_norm"],
           "lm_head": m["lm_head"][1]}
    for i, lw in enumerate(m["layers"]):
        for n in ("attention_norm", "ffn_norm"):
            out[f"l{i}_{n}"] = lw[n]
        for n in O.LINEAR_NAMES:
            out[f"l{i}_{n}"] = lw[n][1]
    out["tokens"] = np.array(TINY_TOKENS, np.int32)
    out["positions"] = np.arange(len(TINY_TOKENS), dtype=np.int32)
    out["logits"] = ref.forward_tokens(m, out["tokens"], out["positions"])
    return out


FIXTURES = (("tiny_chain", tiny_chain), ("quant", quant), ("dequant_kat", dequant_kat),
            ("rows_8b_70b", rows_8b_70b), ("linear", linear), ("attention", attention),
            ("tiny_forward", tiny_forward))


def main():
    ref = O.reference()
    wanted = set(sys.argv[1:])
    for name, fn in FIXTURES:
        if wanted and name not in wanted:
            continue
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn(ref))
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
