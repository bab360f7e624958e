"""Batched forward pass on the device: the reference's ForwardBatch
(src/forward.cc:473-488) without its token loop.  The reference runs each
token of a batch through the whole model (ForwardToken, :432-472); here the
batch goes through each layer at once -- mlk_forward_layer_batch, the
reference's ForwardLayerDevice (:337-384) over [T, dim] -- and only the last
token's logits are computed unless all are asked for (ComputeLogitsDevice,
:425-431).

A model is a dict:
    config      vocab, dim, hidden_dim, layers, n_heads, n_kv_heads,
                head_dim, max_seq, rope_type (0 normal, 1 NeoX), theta, eps
    embedding   [vocab, dim] float32, or
    embedding_q (qtype, blocks): the token table kept as Q8_0 / Q4_0 / Q4_1
                blocks on the device (the reference dequantizes a GGUF
                token_embd to fp32 at load, src/gguf_load.cc:370-404; the
                quantized gather gives the same rows bit for bit)
    layers      per layer: attention_norm, ffn_norm [dim]; wq, wk, wv, wo,
                w_gate, w_up, w_down as ("f32", W [out, in]) or
                (qtype, blocks); optional bq, bk, bv [out]
    final_norm  [dim]
    lm_head     ("f32", W [vocab, dim]) or (qtype, blocks)
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import (DeviceBuffer, QUANT, check, gather_f32, gather_quant, lib, linear_f32,
               linear_quant, quant_planar_bytes, quant_to_planar, rmsnorm)

_i32, _i64, _vp = C.c_int32, C.c_int64, C.c_void_p
WEIGHT_F32 = -1
LINEAR_NAMES = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")


class LayerConfig(C.Structure):
    """mlk_layer_config."""
    _fields_ = [("dim", _i64), ("hidden_dim", _i64), ("n_heads", _i32), ("n_kv_heads", _i32),
                ("head_dim", _i32), ("rope_type", _i32), ("rope_theta", C.c_float),
                ("rms_norm_eps", C.c_float)]


class LinearWeight(C.Structure):
    """mlk_linear_weight."""
    _fields_ = [("type", _i32), ("data", _vp), ("bias", _vp), ("planar", _vp)]


class LayerWeights(C.Structure):
    """mlk_layer_weights."""
    _fields_ = [("attention_norm", _vp), ("wq", LinearWeight), ("wk", LinearWeight),
                ("wv", LinearWeight), ("wo", LinearWeight), ("ffn_norm", _vp),
                ("w_gate", LinearWeight), ("w_up", LinearWeight), ("w_down", LinearWeight)]


lib.mlk_forward_layer_workspace_bytes.restype = _i64
lib.mlk_forward_layer_workspace_bytes.argtypes = [C.POINTER(LayerConfig), _i64, _i64, _i32]
lib.mlk_forward_layer_batch.restype = C.c_int
lib.mlk_forward_layer_batch.argtypes = [C.POINTER(LayerConfig), C.POINTER(LayerWeights), _vp,
                                        _i64, _vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _vp,
                                        C.c_size_t, _vp, _vp]


def layer_config(config):
    return LayerConfig(config["dim"], config["hidden_dim"], config["n_heads"],
                       config["n_kv_heads"], config["head_dim"], config.get("rope_type", 0),
                       config["theta"], config["eps"])


def layer_workspace_bytes(config, n_tokens, max_ctx, consecutive=True):
    cfg = layer_config(config)
    return int(lib.mlk_forward_layer_workspace_bytes(C.byref(cfg), n_tokens, max_ctx,
                                                     1 if consecutive else 0))


def forward_layer_batch(config, weights, x, n_tokens, k_cache, v_cache, n_layers, max_seq, layer,
                        max_ctx, workspace, positions=None, pos0=0, err=None, stream=None):
    """x [n_tokens, dim] (device, in place) through one layer; weights is a
    LayerWeights, workspace a DeviceBuffer of layer_workspace_bytes()."""
    from . import _p, _sp
    cfg = layer_config(config)
    check(lib.mlk_forward_layer_batch(C.byref(cfg), C.byref(weights), _p(x), n_tokens,
                                      _p(positions), pos0, _p(k_cache), _p(v_cache), n_layers,
                                      max_seq, layer, max_ctx, _p(workspace), workspace.nbytes,
                                      _p(err), _sp(stream)),
          "mlk_forward_layer_batch")


class DeviceModel:
    """A model's weights and KV caches on the current device, run through
    batched layers.  The caches persist across calls, as the reference's
    Context does: a prompt chunk, then more chunks or single decode tokens
    at later positions."""

    def __init__(self, model, planar=False):
        """planar: also keep Q8_0 / Q4_0 weights (in_features a multiple of
        256) in the planar layout, which batches of 1..32 tokens run on."""
        c = self.config = dict(model["config"])
        self._keep = []
        self._planar = planar
        if "embedding_q" in model:
            qt, blocks = model["embedding_q"]
            self.embedding = (qt, self._up(np.ascontiguousarray(blocks, np.uint8)))
        else:
            self.embedding = ("f32", self._up(np.ascontiguousarray(model["embedding"],
                                                                   np.float32)))
        self.layers = []
        for lw in model["layers"]:
            w = LayerWeights()
            w.attention_norm = self._up(lw["attention_norm"]).ptr
            w.ffn_norm = self._up(lw["ffn_norm"]).ptr
            QD, KD = c["n_heads"] * c["head_dim"], c["n_kv_heads"] * c["head_dim"]
            shapes = {"wq": (QD, c["dim"]), "wk": (KD, c["dim"]), "wv": (KD, c["dim"]),
                      "wo": (c["dim"], QD), "w_gate": (c["hidden_dim"], c["dim"]),
                      "w_up": (c["hidden_dim"], c["dim"]), "w_down": (c["dim"], c["hidden_dim"])}
            for name in LINEAR_NAMES:
                setattr(w, name, self._linear(lw[name], lw.get("b" + name[1]) if name in
                                              ("wq", "wk", "wv") else None, shapes[name]))
            self.layers.append(w)
        self.final_norm = self._up(model["final_norm"])
        kind, data = model["lm_head"]
        self.lm_head = (kind, self._up(data if kind != "f32" else np.asarray(data, np.float32)))
        L, S, KV, hd = c["layers"], c["max_seq"], c["n_kv_heads"], c["head_dim"]
        self.k_cache = DeviceBuffer.empty((L, S, KV, hd))
        self.v_cache = DeviceBuffer.empty((L, S, KV, hd))
        self.k_cache.zero()
        self.v_cache.zero()
        self._ws = None

    def _up(self, a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.float64:
            a = a.astype(np.float32)
        buf = DeviceBuffer.from_array(a)
        self._keep.append(buf)
        return buf

    def _linear(self, w, bias, shape):
        kind, data = w
        lw = LinearWeight()
        lw.type = WEIGHT_F32 if kind == "f32" else QUANT[kind]
        blocks = self._up(np.asarray(data, np.float32) if kind == "f32" else
                          np.asarray(data, np.uint8))
        lw.data = blocks.ptr
        lw.bias = None if bias is None else self._up(np.asarray(bias, np.float32)).ptr
        n = quant_planar_bytes(kind, *shape) if self._planar and kind in ("q8_0", "q4_0") else 0
        if n > 0:
            planar = DeviceBuffer(n, np.uint8)
            quant_to_planar(kind, blocks, shape[0], shape[1], planar)
            self._keep.append(planar)
            lw.planar = planar.ptr
        return lw

    def _workspace(self, n):
        if self._ws is None or self._ws.nbytes < n:
            if self._ws is not None:
                self._ws.close()
            self._ws = DeviceBuffer(n, np.uint8)
        return self._ws

    def embed(self, tokens, out, stream=None):
        c = self.config
        ids = DeviceBuffer.from_array(np.ascontiguousarray(tokens, np.int32))
        kind, table = self.embedding
        if kind == "f32":
            gather_f32(table, c["vocab"], c["dim"], ids, len(tokens), out, stream=stream)
        else:
            gather_quant(kind, table, c["vocab"], c["dim"], ids, len(tokens), out, stream=stream)

    def hidden(self, tokens, positions=None, pos0=0, stream=None, err=None):
        """The residual stream after the last layer, [T, dim] on the device."""
        c = self.config
        T = len(tokens)
        x = DeviceBuffer.empty((T, c["dim"]))
        self.embed(tokens, x, stream)
        d_pos = None
        if positions is not None:
            positions = np.ascontiguousarray(positions, np.int32)
            d_pos = DeviceBuffer.from_array(positions)
            max_ctx = int(positions.max()) + 1
        else:
            max_ctx = pos0 + T
        ws = self._workspace(layer_workspace_bytes(c, T, max_ctx, positions is None))
        for li, w in enumerate(self.layers):
            forward_layer_batch(c, w, x, T, self.k_cache, self.v_cache, c["layers"],
                                c["max_seq"], li, max_ctx, ws, positions=d_pos, pos0=pos0,
                                err=err, stream=stream)
        return x

    def logits(self, x, rows, stream=None):
        """Final RmsNorm and lm_head over `rows` rows of x [T, dim] starting at
        row T - rows (ComputeLogitsDevice on each)."""
        c = self.config
        D, V = c["dim"], c["vocab"]
        T = x.shape[0]
        src = x.ptr + (T - rows) * D * 4
        h = DeviceBuffer.empty((rows, D))
        rmsnorm(src, self.final_norm, h, rows, D, c["eps"], stream=stream)
        out = DeviceBuffer.empty((rows, V))
        kind, w = self.lm_head
        if kind == "f32":
            linear_f32(h, w, out, rows, D, V, stream=stream)
        else:
            linear_quant(kind, h, w, out, rows, D, V, stream=stream)
        return out

    def forward(self, tokens, positions=None, pos0=0, all_logits=False, stream=None):
        """ForwardBatch: the logits of the last token ([vocab]) or of every
        token ([T, vocab]) as numpy."""
        x = self.hidden(tokens, positions, pos0, stream)
        out = self.logits(x, len(tokens) if all_logits else 1, stream)
        res = out.download()
        return res if all_logits else res[0]
