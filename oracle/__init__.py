"""ctypes bindings for the CPU oracle (liboracle.so) and the compiled reference
(oracle/_ref/libref*.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker and by bench.py's cpu_baseline leg.  The product package never
imports this module.

Arrays are numpy arrays; every wrapper checks dtype and contiguity and raises
ValueError when the C function reports ORC_EINVAL (the input the reference
would throw on).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# MLK_ORACLE_LIB selects another build of the same source (the sanitizer test
# runs the oracle tests against an AddressSanitizer + UBSan build)
ORACLE_SO = os.environ.get("MLK_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")
REF_AVX2_SO = os.path.join(HERE, "_ref", "libref_avx2.so")

QUANT_TYPES = {"q8_0": 0, "q4_0": 1, "q4_1": 2}
BLOCK_BYTES = {"q8_0": 34, "q4_0": 18, "q4_1": 20}
ROPE_NORMAL, ROPE_NEOX = 0, 1

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64 = C.c_int64
_i32 = C.c_int32


def _bind(lib, name, restype, argtypes):
    fn = getattr(lib, name)
    fn.restype = restype
    fn.argtypes = argtypes
    return fn


class _Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built; run `make -C oracle`")
        lib = C.CDLL(path)
        self.lib = lib
        self.fp16_to_fp32 = _bind(lib, "orc_fp16_to_fp32", C.c_float, [C.c_uint16])
        self.fp32_to_fp16 = _bind(lib, "orc_fp32_to_fp16", C.c_uint16, [C.c_float])
        _u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
        self._h2f = _bind(lib, "orc_fp16_to_fp32_array", None, [_u16p, _f32p, _i64])
        self._f2h = _bind(lib, "orc_fp32_to_fp16_array", None, [_f32p, _u16p, _i64])
        for q in QUANT_TYPES:
            setattr(self, f"_quantize_{q}",
                    _bind(lib, f"orc_quantize_{q}", C.c_int, [_f32p, _i64, _i64, _u8p]))
            setattr(self, f"_dequantize_{q}",
                    _bind(lib, f"orc_dequantize_{q}", C.c_int, [_u8p, _i64, _i64, _f32p]))
        self._gather_f32 = _bind(lib, "orc_gather_f32", C.c_int,
                                 [_f32p, _i64, _i64, _i32p, _i64, _f32p])
        self._gather_quant = _bind(lib, "orc_gather_quant", C.c_int,
                                   [C.c_int, _u8p, _i64, _i64, _i32p, _i64, _f32p])
        for name in ("add", "mul", "swiglu"):
            setattr(self, f"_{name}", _bind(lib, f"orc_{name}", None, [_f32p, _f32p, _f32p, _i64]))
        self._silu = _bind(lib, "orc_silu", None, [_f32p, _f32p, _i64])
        self._softmax = _bind(lib, "orc_softmax", C.c_int, [_f32p, _f32p, _i64])
        self._rmsnorm_row = _bind(lib, "orc_rmsnorm_row", C.c_int,
                                  [_f32p, _f32p, _f32p, _i64, C.c_float])
        self._add_rmsnorm = _bind(lib, "orc_add_rmsnorm", C.c_int,
                                  [_f32p, C.c_void_p, _f32p, _f32p, _i64, _i64, C.c_float])
        self._rope = _bind(lib, "orc_rope", C.c_int,
                           [_f32p, _f32p, _i64, _i32, _i32, _i32, C.c_void_p, _i32,
                            C.c_float, _i32])
        self._chain = _bind(lib, "orc_chain", C.c_int,
                            [_f32p, _i64, _i64, _i32p, _f32p, _f32p, _f32p, _f32p, C.c_float,
                             _f32p, _f32p, _i32, _i32, _i32, _i32p, C.c_float,
                             _f32p, _f32p, _f32p, _i64, _i64, C.c_int])
        self.parallel_threads = _bind(lib, "orc_parallel_threads", C.c_int, [C.c_int])
        self._linear_quant = _bind(lib, "orc_linear_quant", C.c_int,
                                   [C.c_int, _f32p, _u8p, C.c_void_p, _f32p, _i64, _i64, _i64,
                                    C.c_int])
        self._linear_f32 = _bind(lib, "orc_linear_f32", C.c_int,
                                 [_f32p, _f32p, C.c_void_p, _f32p, _i64, _i64, _i64, C.c_int])
        self._matmul_f32 = _bind(lib, "orc_matmul_f32", C.c_int,
                                 [_f32p, _f32p, _f32p, _i64, _i64, _i64, C.c_int])
        self._kv_write = _bind(lib, "orc_kv_write", C.c_int,
                               [_f32p, _f32p, _i64, _i64, _i32, _i32, _i64, _i32p, _i64, _f32p,
                                _f32p])
        self._attention = _bind(lib, "orc_attention", C.c_int,
                                [_f32p, _f32p, _f32p, _i64, _i64, _i32, _i32, _i32, _i64, _i32p,
                                 _i64, _f32p])

    # ---- attention and KV cache ----------------------------------------------
    def kv_write(self, k_cache, v_cache, layer, positions, k, v):
        """Writes k, v [T, KV, hd] into slots (layer, positions[t]) of the caches
        [L, S, KV, hd] in place."""
        L, S, KV, hd = k_cache.shape
        pos = np.ascontiguousarray(positions, dtype=np.int32)
        _check(self._kv_write(k_cache.reshape(-1), v_cache.reshape(-1), L, S, KV, hd, layer, pos,
                              pos.size, _f32(k).reshape(-1), _f32(v).reshape(-1)))

    def attention(self, q, k_cache, v_cache, layer, positions):
        """out [T, H, hd] for q [T, H, hd] against caches [L, S, KV, hd]."""
        q = _f32(q)
        L, S, KV, hd = k_cache.shape
        T, H = q.shape[0], q.shape[1]
        pos = np.ascontiguousarray(positions, dtype=np.int32)
        out = np.empty((T, H, hd), np.float32)
        _check(self._attention(q.reshape(-1), _f32(k_cache).reshape(-1), _f32(v_cache).reshape(-1),
                               L, S, H, KV, hd, layer, pos, T, out.reshape(-1)))
        return out

    def fp16_to_fp32_array(self, codes):
        codes = np.ascontiguousarray(codes, dtype=np.uint16)
        out = np.empty(codes.shape, np.float32)
        self._h2f(codes.reshape(-1), out.reshape(-1), codes.size)
        return out

    def fp32_to_fp16_array(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape, np.uint16)
        self._f2h(x.reshape(-1), out.reshape(-1), x.size)
        return out

    # ---- quant -------------------------------------------------------------
    def quantize(self, qtype, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, cols = (1, x.shape[0]) if x.ndim == 1 else (int(np.prod(x.shape[:-1])), x.shape[-1])
        nb = (cols + 31) // 32
        out = np.zeros(rows * nb * BLOCK_BYTES[qtype], dtype=np.uint8)
        _check(getattr(self, f"_quantize_{qtype}")(x.reshape(-1), rows, cols, out))
        return out

    def dequantize(self, qtype, blocks, rows, cols):
        out = np.zeros(rows * cols, dtype=np.float32)
        _check(getattr(self, f"_dequantize_{qtype}")(_u8(blocks), rows, cols, out))
        return out.reshape(rows, cols)

    # ---- gather ------------------------------------------------------------
    def gather_f32(self, table, ids):
        table = _f32(table)
        vocab, dim = table.shape
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.zeros((len(ids), dim), dtype=np.float32)
        _check(self._gather_f32(table.reshape(-1), vocab, dim, ids, len(ids), out.reshape(-1)))
        return out

    def gather_quant(self, qtype, blocks, vocab, dim, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.zeros((len(ids), dim), dtype=np.float32)
        _check(self._gather_quant(QUANT_TYPES[qtype], _u8(blocks), vocab, dim, ids, len(ids),
                                  out.reshape(-1)))
        return out

    # ---- elementwise -------------------------------------------------------
    def _binary(self, fn, a, b):
        a, b = _f32(a), _f32(b)
        if a.shape != b.shape:
            raise ValueError("shapes must match")
        y = np.empty_like(a)
        fn(a.reshape(-1), b.reshape(-1), y.reshape(-1), a.size)
        return y

    def add(self, a, b):
        return self._binary(self._add, a, b)

    def mul(self, a, b):
        return self._binary(self._mul, a, b)

    def swiglu(self, gate, up):
        return self._binary(self._swiglu, gate, up)

    def silu(self, x):
        x = _f32(x)
        y = np.empty_like(x)
        self._silu(x.reshape(-1), y.reshape(-1), x.size)
        return y

    def softmax(self, x):
        x = _f32(x)
        y = np.empty_like(x)
        _check(self._softmax(x.reshape(-1), y.reshape(-1), x.size))
        return y

    # ---- rmsnorm -----------------------------------------------------------
    def rmsnorm(self, x, w, eps):
        """Row-wise RmsNorm of a [rows, dim] (or [dim]) array."""
        x = _f32(x)
        r = x.copy()
        y = np.empty_like(x)
        dim = x.shape[-1]
        _check(self._add_rmsnorm(r.reshape(-1), None, _f32(w), y.reshape(-1), x.size // dim, dim,
                                 eps))
        return y

    def add_rmsnorm(self, residual, delta, w, eps):
        """Returns (residual + delta, RmsNorm(residual + delta)) row-wise."""
        r = _f32(residual).copy()
        delta = _f32(delta)
        y = np.empty_like(r)
        dim = r.shape[-1]
        _check(self._add_rmsnorm(r.reshape(-1), delta.ctypes.data, _f32(w), y.reshape(-1),
                                 r.size // dim, dim, eps))
        return r, y

    # ---- rope --------------------------------------------------------------
    def rope(self, q, k, n_heads, n_kv_heads, head_dim, positions=None, pos0=0,
             theta=10000.0, rope_type=ROPE_NORMAL):
        """Returns rotated copies of q [T, H*hd] and k [T, KV*hd]."""
        q = _f32(q).copy()
        k = _f32(k).copy()
        n_tokens = q.size // (n_heads * head_dim)
        pos_arr = None
        ptr = None
        if positions is not None:
            pos_arr = np.ascontiguousarray(positions, dtype=np.int32)
            ptr = pos_arr.ctypes.data
        _check(self._rope(q.reshape(-1), k.reshape(-1), n_tokens, n_heads, n_kv_heads, head_dim,
                          ptr, pos0, theta, rope_type))
        return q, k

    # ---- linear ------------------------------------------------------------
    def linear_quant(self, qtype, x, blocks, out_features, bias=None, n_threads=0):
        """y = x @ dequant(W)^T (+ bias) for x [rows, in] (or [in])."""
        x = _f32(x)
        rows, in_f = (1, x.shape[0]) if x.ndim == 1 else x.shape
        y = np.empty((rows, out_features), np.float32)
        b = None if bias is None else _f32(bias)
        _check(self._linear_quant(QUANT_TYPES[qtype], x.reshape(-1), _u8(blocks),
                                  None if b is None else b.ctypes.data, y.reshape(-1), rows, in_f,
                                  out_features, n_threads))
        return y.reshape(-1) if x.ndim == 1 else y

    def linear_f32(self, x, w, bias=None, n_threads=0):
        """y = x @ W^T (+ bias), W [out, in]."""
        x, w = _f32(x), _f32(w)
        rows, in_f = (1, x.shape[0]) if x.ndim == 1 else x.shape
        y = np.empty((rows, w.shape[0]), np.float32)
        b = None if bias is None else _f32(bias)
        _check(self._linear_f32(x.reshape(-1), w.reshape(-1), None if b is None else b.ctypes.data,
                                y.reshape(-1), rows, in_f, w.shape[0], n_threads))
        return y.reshape(-1) if x.ndim == 1 else y

    def matmul_f32(self, a, b, n_threads=0):
        a, b = _f32(a), _f32(b)
        c = np.empty((a.shape[0], b.shape[1]), np.float32)
        _check(self._matmul_f32(a.reshape(-1), b.reshape(-1), c.reshape(-1), a.shape[0],
                                a.shape[1], b.shape[1], n_threads))
        return c

    # ---- CPU baseline ------------------------------------------------------
    def chain(self, bufs, n_tokens, n_threads):
        return self._chain(*_chain_args(bufs, n_tokens, n_threads))

    # ---- forward pass ------------------------------------------------------
    def linear(self, w, x, out_features, bias=None):
        """A model linear: w = ("f32", W [out, in]) or (qtype, blocks)."""
        kind, data = w
        if kind == "f32":
            return self.linear_f32(x, data, bias)
        return self.linear_quant(kind, x, data, out_features, bias)

    def layer_token(self, c, lw, x, kc, vc, li, pos, mistake=None, keep=None):
        """One layer of ForwardLayer (src/forward.cc:385-414) for one token
        at `pos`: x [dim] in, the layer's output out; its K/V row is written
        to slot (li, pos) of kc / vc [layers, max_seq, KV, hd] first, and
        the token attends to slots 0..pos.  keep: a dict that receives the
        intermediates (h, q, k, v after RoPE, a, r, h2, f)."""
        D, H, KV, hd = c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"]
        F = c["hidden_dim"]
        h = self.rmsnorm(x, lw["ffn_norm" if mistake == "swap_norms" else "attention_norm"],
                         c["eps"])
        q = self.linear(lw["wq"], h, H * hd, lw.get("bq"))
        k = self.linear(lw["wk"], h, KV * hd, lw.get("bk"))
        v = self.linear(lw["wv"], h, KV * hd, lw.get("bv"))
        if mistake != "no_rope_on_k":
            q, k = self.rope(q[None], k[None], H, KV, hd, positions=[pos],
                             theta=c["theta"], rope_type=c["rope_type"])
        else:
            q, _ = self.rope(q[None], k[None], H, KV, hd, positions=[pos],
                             theta=c["theta"], rope_type=c["rope_type"])
            k = k[None]
        self.kv_write(kc, vc, li, [pos], k.reshape(1, KV, hd), v.reshape(1, KV, hd))
        a = self.attention(q.reshape(1, H, hd), kc, vc, li,
                           [pos - 1 if mistake == "exclusive_attention" and pos > 0 else pos])
        o = self.linear(lw["wo"], a.reshape(-1), D)
        r = x if mistake == "no_attention_residual" else self.add(x, o)
        if mistake == "no_attention_residual":
            r = o
        h2 = self.rmsnorm(r, lw["ffn_norm"], c["eps"])
        g = self.linear(lw["w_gate"], h2, F)
        u = self.linear(lw["w_up"], h2, F)
        f = self.swiglu(u, g) if mistake == "swap_gate_up" else self.swiglu(g, u)
        if keep is not None:
            keep.update(h=h, q=np.ravel(q), k=np.ravel(k), v=np.ravel(v), a=np.ravel(a), r=r,
                        h2=h2, f=f)
        return self.add(r, self.linear(lw["w_down"], f, D))

    def layer_tokens(self, c, lw, x, kc, vc, li, positions, keep=None):
        """ForwardBatch's token loop (src/forward.cc:482-486) restricted to
        one layer: rows t of x [T, dim] in order, token t at positions[t]
        over the caches as they stand (already-filled slots included);
        returns the layer's outputs [T, dim] and updates the caches.  keep:
        a list that receives each token's intermediates (layer_token)."""
        x = np.asarray(x, np.float32)
        out = []
        for t in range(x.shape[0]):
            d = {} if keep is not None else None
            out.append(self.layer_token(c, lw, x[t], kc, vc, li, int(positions[t]), keep=d))
            if keep is not None:
                keep.append(d)
        return np.stack(out)

    def forward_tokens(self, model, tokens, positions, mistake=None):
        """The reference's CPU forward pass restated over the ops above:
        ForwardBatch's loop (src/forward.cc:473-488) of ForwardToken
        (:432-472) for tokens[t] at positions[t], one token at a time over
        one KV cache:
          x = Embedding(token)                               :198-205
          per layer (ForwardLayer :385-414):
            h = RmsNorm(x, attention_norm)
            q, k, v = Linear(h, wq / wk / wv) + optional bias  :328-336, 223-236
            Rope(q, k, pos)
            write k, v at pos; a = ForwardAttention            :265-298
            r = x + Linear(a, wo)                              :213-222
            h2 = RmsNorm(r, ffn_norm)
            x = r + Linear(SwiGlu(Linear(h2, w_gate), Linear(h2, w_up)), w_down)
          logits = Linear(RmsNorm(x, final_norm), lm_head)   ComputeLogits :415-424
        model: forward_model() layout.  Returns (logits [T, vocab], hidden
        [T, layers + 1, dim]: the residual stream entering each layer and
        leaving the last).  `mistake` plants one error, for the tests that
        show the pinning catches it."""
        c = model["config"]
        D, H, KV, hd = c["dim"], c["n_heads"], c["n_kv_heads"], c["head_dim"]
        L, F, V = c["layers"], c["hidden_dim"], c["vocab"]
        kc = np.zeros((L, c["max_seq"], KV, hd), np.float32)
        vc = np.zeros_like(kc)
        T = len(tokens)
        logits = np.empty((T, V), np.float32)
        hidden = np.empty((T, L + 1, D), np.float32)
        for t in range(T):
            pos = int(positions[t])
            if "embedding" in model:
                x = self.gather_f32(model["embedding"], np.array([tokens[t]], np.int32))[0]
            else:
                qt, blocks = model["embedding_q"]
                x = self.gather_quant(qt, blocks, V, D, np.array([tokens[t]], np.int32))[0]
            for li, lw in enumerate(model["layers"]):
                hidden[t, li] = x
                x = self.layer_token(c, lw, x, kc, vc, li, pos, mistake)
            hidden[t, L] = x
            logits[t] = self.linear(model["lm_head"], self.rmsnorm(x, model["final_norm"],
                                                                   c["eps"]), V)
        return logits, hidden


LINEAR_NAMES = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")
FORWARD_MISTAKES = ("swap_norms", "no_rope_on_k", "exclusive_attention", "no_attention_residual",
                    "swap_gate_up")


def linear_shapes(c):
    """[out, in] of each layer linear for a forward_model config."""
    D, F = c["dim"], c["hidden_dim"]
    QD, KD = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
    return {"wq": (QD, D), "wk": (KD, D), "wv": (KD, D), "wo": (D, QD), "w_gate": (F, D),
            "w_up": (F, D), "w_down": (D, F)}


def forward_model(config, seed, weight_type="f32", biases=False, quant_embedding=None,
                  std=0.02):
    """A random model in the layout forward_tokens takes: config keys vocab,
    dim, hidden_dim, layers, n_heads, n_kv_heads, head_dim, max_seq,
    rope_type, theta, eps; weights N(0, std) (norm weights N(1, 0.1)),
    quantized by the restated quantizer when weight_type is a qtype;
    quant_embedding: a qtype to keep the token table as blocks."""
    rng = np.random.default_rng(seed)
    orc = oracle()
    c = dict(config)

    def lin(out_f, in_f):
        w = (rng.standard_normal((out_f, in_f)) * std).astype(np.float32)
        return ("f32", w) if weight_type == "f32" else (weight_type, orc.quantize(weight_type, w))

    model = {"config": c, "layers": []}
    table = (rng.standard_normal((c["vocab"], c["dim"])) * std).astype(np.float32)
    if quant_embedding:
        model["embedding_q"] = (quant_embedding, orc.quantize(quant_embedding, table))
    else:
        model["embedding"] = table
    for _ in range(c["layers"]):
        lw = {"attention_norm": (1 + 0.1 * rng.standard_normal(c["dim"])).astype(np.float32),
              "ffn_norm": (1 + 0.1 * rng.standard_normal(c["dim"])).astype(np.float32)}
        for name, (o, i) in linear_shapes(c).items():
            lw[name] = lin(o, i)
        if biases:
            for b, n in (("bq", "wq"), ("bk", "wk"), ("bv", "wv")):
                lw[b] = (rng.standard_normal(linear_shapes(c)[n][0]) * 0.1).astype(np.float32)
        model["layers"].append(lw)
    model["final_norm"] = (1 + 0.1 * rng.standard_normal(c["dim"])).astype(np.float32)
    model["lm_head"] = lin(c["vocab"], c["dim"])
    return model


def _chain_args(b, n_tokens, n_threads):
    return (b["table"].reshape(-1), b["vocab"], b["dim"], b["ids"], b["x"].reshape(-1),
            b["delta"].reshape(-1), b["norm_w"], b["y"].reshape(-1), b["eps"],
            b["q"].reshape(-1), b["k"].reshape(-1), b["n_heads"], b["n_kv_heads"],
            b["head_dim"], b["positions"], b["theta"], b["gate"].reshape(-1),
            b["up"].reshape(-1), b["ffn_out"].reshape(-1), b["ffn_dim"], n_tokens, n_threads)


class _Reference:
    """The reference's own CPU code (oracle/_ref), built from its sources."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built (needs the reference tree)")
        lib = C.CDLL(path)
        self.path = path
        self._rmsnorm_row = _bind(lib, "ref_rmsnorm_row", C.c_int,
                                  [_f32p, _f32p, _f32p, C.c_int, C.c_float])
        self._rope_token = _bind(lib, "ref_rope_token", C.c_int,
                                 [_f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                  C.c_int])
        self._silu = _bind(lib, "ref_silu", C.c_int, [_f32p, _f32p, C.c_int])
        self._mul = _bind(lib, "ref_mul", C.c_int, [_f32p, _f32p, _f32p, C.c_int])
        self._swiglu = _bind(lib, "ref_swiglu", C.c_int, [_f32p, _f32p, _f32p, C.c_int])
        self._softmax = _bind(lib, "ref_softmax", C.c_int, [_f32p, _f32p, C.c_int])
        self._quantize = _bind(lib, "ref_quantize", C.c_int,
                               [C.c_int, _f32p, C.c_int, C.c_int, _u8p])
        self._dequantize = _bind(lib, "ref_dequantize", C.c_int,
                                 [C.c_int, _u8p, C.c_int, C.c_int, _f32p])
        self._dequantize_flat = _bind(lib, "ref_dequantize_flat", C.c_int,
                                      [C.c_int, _u8p, C.c_int, C.c_int, _f32p])
        vp = C.c_void_p
        self._chain = _bind(lib, "ref_chain", C.c_int,
                            [vp, _i32p, vp, _f32p, _f32p, _f32p, _f32p, C.c_float,
                             _f32p, _f32p, C.c_int, C.c_int, C.c_int, _i32p, C.c_float,
                             _f32p, _f32p, _f32p, _i64, _i64, _i64, C.c_int])
        self._embedding_model = _bind(lib, "ref_embedding_model", vp, [_f32p, _i64, _i64])
        self._model_free = _bind(lib, "ref_model_free", None, [vp])
        self._gather_quant = _bind(lib, "ref_gather_quant", C.c_int,
                                   [C.c_int, _u8p, _i64, _i64, _i32p, _i64, _f32p, C.c_int])
        self._linear_quant = _bind(lib, "ref_linear_quant", C.c_int,
                                   [C.c_int, _f32p, _u8p, _f32p, C.c_int, C.c_int, C.c_int,
                                    C.c_int])
        self._linear_f32 = _bind(lib, "ref_linear_f32", C.c_int,
                                 [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int])
        self._matmul_f32 = _bind(lib, "ref_matmul_f32", C.c_int,
                                 [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int])
        self._attention = _bind(lib, "ref_attention", C.c_int,
                                [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                 C.c_int, C.c_int, _f32p])
        vp = C.c_void_p
        self._forward_tokens = _bind(lib, "ref_forward_tokens", C.c_int,
                                     [_i32p, C.c_float, C.c_float, _f32p, C.POINTER(vp), _i32p,
                                      C.POINTER(vp), C.POINTER(vp), _f32p, _i32p, _i32p, C.c_int,
                                      _f32p])

    def attention(self, q, k_rows, v_rows, n_layers, max_seq, layer, pos):
        """One query token q [H, hd] at `pos`: k_rows / v_rows [pos + 1, KV, hd]
        are written to the reference's own KvCache (src/kvcache.cc) slots
        0..pos of `layer`, then the ForwardAttention loop runs over it."""
        q = _f32(q)
        H, hd = q.shape
        KV = k_rows.shape[1]
        out = np.empty((H, hd), np.float32)
        _check(self._attention(q.reshape(-1), _f32(k_rows).reshape(-1), _f32(v_rows).reshape(-1),
                               n_layers, max_seq, H, KV, hd, layer, pos, out.reshape(-1)))
        return out

    def linear_quant(self, qtype, x, blocks, out_features, n_threads=0):
        x = _f32(x)
        rows, in_f = (1, x.shape[0]) if x.ndim == 1 else x.shape
        y = np.empty((rows, out_features), np.float32)
        _check(self._linear_quant(QUANT_TYPES[qtype], x.reshape(-1), _u8(blocks), y.reshape(-1),
                                  rows, in_f, out_features, n_threads))
        return y.reshape(-1) if x.ndim == 1 else y

    def linear_f32(self, x, w):
        x, w = _f32(x), _f32(w)
        rows, in_f = (1, x.shape[0]) if x.ndim == 1 else x.shape
        y = np.empty((rows, w.shape[0]), np.float32)
        _check(self._linear_f32(x.reshape(-1), w.reshape(-1), y.reshape(-1), rows, in_f,
                                w.shape[0]))
        return y.reshape(-1) if x.ndim == 1 else y

    def matmul_f32(self, a, b):
        a, b = _f32(a), _f32(b)
        c = np.empty((a.shape[0], b.shape[1]), np.float32)
        _check(self._matmul_f32(a.reshape(-1), b.reshape(-1), c.reshape(-1), a.shape[0],
                                a.shape[1], b.shape[1]))
        return c

    def rmsnorm_row(self, x, w, eps):
        x = _f32(x)
        y = np.empty_like(x)
        _check(self._rmsnorm_row(x, _f32(w), y, x.size, eps))
        return y

    def rope_token(self, q, k, n_heads, n_kv_heads, head_dim, pos, theta, rope_type=ROPE_NORMAL):
        q = _f32(q).copy()
        k = _f32(k).copy()
        _check(self._rope_token(q.reshape(-1), k.reshape(-1), n_heads, n_kv_heads, head_dim, pos,
                                theta, rope_type))
        return q, k

    def silu(self, x):
        x = _f32(x)
        y = np.empty_like(x)
        _check(self._silu(x.reshape(-1), y.reshape(-1), x.size))
        return y

    def mul(self, a, b):
        a, b = _f32(a), _f32(b)
        y = np.empty_like(a)
        _check(self._mul(a.reshape(-1), b.reshape(-1), y.reshape(-1), a.size))
        return y

    def swiglu(self, g, u):
        g, u = _f32(g), _f32(u)
        y = np.empty_like(g)
        _check(self._swiglu(g.reshape(-1), u.reshape(-1), y.reshape(-1), g.size))
        return y

    def softmax(self, x):
        x = _f32(x)
        y = np.empty_like(x)
        _check(self._softmax(x.reshape(-1), y.reshape(-1), x.size))
        return y

    def quantize(self, qtype, x):
        x = _f32(x)
        rows, cols = (1, x.shape[0]) if x.ndim == 1 else (int(np.prod(x.shape[:-1])), x.shape[-1])
        out = np.zeros(rows * ((cols + 31) // 32) * BLOCK_BYTES[qtype], dtype=np.uint8)
        _check(self._quantize(QUANT_TYPES[qtype], x.reshape(-1), rows, cols, out))
        return out

    def dequantize(self, qtype, blocks, rows, cols, flat=False):
        out = np.zeros(rows * cols, dtype=np.float32)
        fn = self._dequantize_flat if flat else self._dequantize
        _check(fn(QUANT_TYPES[qtype], _u8(blocks), rows, cols, out))
        return out.reshape(rows, cols)

    def embedding_model(self, table):
        """A reference Model holding only the F32 token table (one copy);
        free it with free_model."""
        table = _f32(table)
        handle = self._embedding_model(table.reshape(-1), table.shape[0], table.shape[1])
        if not handle:
            raise MemoryError("ref_embedding_model failed")
        return handle

    def free_model(self, handle):
        self._model_free(handle)

    def chain(self, bufs, n_tokens, n_threads):
        """The chain over the reference's own Embedding, ForwardAdd, RmsNorm,
        Rope and SwiGlu (ref_chain).  bufs as for the oracle's chain; a
        bufs["model"] handle (embedding_model) is used as it is, else one is
        made from bufs["table"] for the call.  bufs["table"] None means no
        gather: bufs["x_in"] rows are the residual input."""
        b = bufs
        model, own = b.get("model"), False
        if model is None and b.get("table") is not None:
            model, own = self.embedding_model(b["table"]), True
        try:
            x_in = None if model is not None else _f32(b["x_in"]).ctypes.data
            ids = b["ids"] if model is not None else np.zeros(1, np.int32)
            return self._chain(model, ids, x_in,
                               b["x"].reshape(-1), b["delta"].reshape(-1), b["norm_w"],
                               b["y"].reshape(-1), b["eps"], b["q"].reshape(-1),
                               b["k"].reshape(-1), b["n_heads"], b["n_kv_heads"], b["head_dim"],
                               b["positions"], b["theta"], b["gate"].reshape(-1),
                               b["up"].reshape(-1), b["ffn_out"].reshape(-1), b["dim"],
                               b["ffn_dim"], n_tokens, n_threads)
        finally:
            if own:
                self.free_model(model)

    def gather_quant(self, qtype, blocks, vocab, dim, ids, n_threads=1):
        """Rows ids of a block-quantized table through the reference's own
        Q*ToTensor (ref_gather_quant); returns [T, dim]."""
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty((ids.size, dim), np.float32)
        _check(self._gather_quant(QUANT_TYPES[qtype], _u8(blocks), vocab, dim, ids, ids.size,
                                  out.reshape(-1), n_threads))
        return out

    def forward_tokens(self, model, tokens, positions):
        """The reference's own ForwardToken loop (ref_forward_tokens) over a
        forward_model(); returns logits [T, vocab].  The F32 token table
        only: the reference dequantizes a quantized one at load."""
        c = model["config"]
        keep = []

        def ptr(a):
            if a is None:
                return None
            keep.append(a)
            return a.ctypes.data

        cfg = np.array([c["vocab"], c["dim"], c["hidden_dim"], c["layers"], c["n_heads"],
                        c["n_kv_heads"], c["head_dim"], c["max_seq"], c["rope_type"]], np.int32)
        norms, types, weights, biases = [], [], [], []
        kinds = {"f32": -1, **QUANT_TYPES}
        for lw in model["layers"]:
            norms += [ptr(_f32(lw["attention_norm"])), ptr(_f32(lw["ffn_norm"]))]
            for name in LINEAR_NAMES:
                kind, data = lw[name]
                types.append(kinds[kind])
                weights.append(ptr(_f32(data) if kind == "f32" else _u8(data)))
            for b in ("bq", "bk", "bv"):
                biases.append(ptr(None if lw.get(b) is None else _f32(lw[b])))
        kind, data = model["lm_head"]
        types.append(kinds[kind])
        weights.append(ptr(_f32(data) if kind == "f32" else _u8(data)))
        vp = C.c_void_p
        n_w = len(weights)
        logits = np.empty((len(tokens), c["vocab"]), np.float32)
        emb = _f32(model["embedding"])
        fn = self._forward_tokens
        _check(fn(cfg, c["theta"], c["eps"], emb, (vp * len(norms))(*norms),
                  np.array(types, np.int32), (vp * n_w)(*weights),
                  (vp * len(biases))(*biases), _f32(model["final_norm"]),
                  np.ascontiguousarray(tokens, np.int32),
                  np.ascontiguousarray(positions, np.int32), len(tokens), logits.reshape(-1)))
        return logits


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8).reshape(-1)


def _check(rc):
    if rc != 0:
        raise ValueError(f"oracle rejected the input (status {rc})")


_oracle = None
_reference = {}


def oracle() -> _Oracle:
    """The C restatement; raises FileNotFoundError if liboracle.so is missing."""
    global _oracle
    if _oracle is None:
        _oracle = _Oracle()
    return _oracle


def reference(avx2: bool = False) -> _Reference:
    """The compiled reference; raises FileNotFoundError when it is not built."""
    path = REF_AVX2_SO if avx2 else REF_SO
    if path not in _reference:
        _reference[path] = _Reference(path)
    return _reference[path]


def reference_available(avx2: bool = False) -> bool:
    return os.path.exists(REF_AVX2_SO if avx2 else REF_SO)
