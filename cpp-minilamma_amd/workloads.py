"""Benchmark configurations and algorithmic byte counts.

The five configurations of BASELINE.json (`configs[0..4]`), the token-id
generator, and the per-op algorithmic HBM bytes used for GB/s and roofline
fractions.  Pure Python + numpy; no GPU needed.
"""
from __future__ import annotations

import numpy as np

HBM_PEAK_GBS = 8000.0  # MI355X published HBM3E bandwidth, GB/s

LLAMA3_8B = dict(vocab=128256, dim=4096, n_heads=32, n_kv_heads=8, head_dim=128, ffn=14336,
                 theta=500000.0, eps=1e-5)
LLAMA3_70B = dict(dim=8192, n_heads=64, n_kv_heads=8, head_dim=128, ffn=28672, theta=500000.0,
                  eps=1e-5)

CONFIGS = {
    # tiny-model op chain (the reference's CPU-runnable case)
    # (table N(0, 0.02), norm weight N(1, 0.1), activations and the residual
    # delta N(0, 1): act_std; the 8B and 70B configs scale activations by 0.02)
    "c1_tiny": dict(vocab=131, dim=64, n_heads=4, n_kv_heads=2, head_dim=16, ffn=172,
                    eps=1e-5, theta=10000.0, ids=[128, 104, 101, 108, 108, 111], seed=42,
                    act_std=1.0),
    # 8B decode step, T = 1..64, positions uniform in [0, 8191]
    "c2_decode_8b": dict(LLAMA3_8B, tokens=(1, 2, 4, 8, 16, 32, 64), max_pos=8191, seed=42),
    # 8B prefill, T = 4096 at positions 0..4095
    "c3_prefill_8b": dict(LLAMA3_8B, tokens=4096, seed=42),
    # quantized embedding gather, T = 4096 Zipf(1.1) ids, seed 7
    "c4_quant_gather": dict(vocab=128256, dim=4096, tokens=4096, seed=7),
    # 70B single-layer op chain, T = 8192
    "c5_70b": dict(LLAMA3_70B, tokens=8192, seed=11),
}

BLOCK_BYTES = {"q8_0": 34, "q4_0": 18, "q4_1": 20}


def zipf_ids(n, vocab, s=1.1, seed=7):
    """n token ids from a Zipf(s) law truncated to [0, vocab): id r has
    probability proportional to (r + 1)^-s (inverse CDF over ranks)."""
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    cdf = np.cumsum(ranks ** -s)
    cdf /= cdf[-1]
    u = np.random.default_rng(seed).random(n)
    return np.minimum(np.searchsorted(cdf, u, side="right"), vocab - 1).astype(np.int32)


def decode_positions(n, max_pos=8191, seed=42):
    return np.random.default_rng(seed).integers(0, max_pos + 1, size=n).astype(np.int32)


# ---------------------------------------------------- algorithmic bytes
# fp32 traffic each op must move at least once, per call.

def bytes_add_rmsnorm(T, D):
    """read x, delta, w; write x', y"""
    return 16 * T * D + 4 * D


def bytes_rmsnorm(T, D):
    return 8 * T * D + 4 * D


def bytes_swiglu(T, F):
    return 12 * T * F


def bytes_rope(T, H, KV, hd):
    return 8 * T * (H + KV) * hd


def bytes_gather_f32(T, D):
    return 8 * T * D + 4 * T


def bytes_gather_quant(qtype, T, D):
    return T * (-(-D // 32) * BLOCK_BYTES[qtype] + 4 * D) + 4 * T


def bytes_gather_unique(ids, D, qtype=None):
    """Bytes a gather must move when every distinct row is read once (a
    Zipf(1.1) batch repeats hot rows, which then come from cache): distinct
    rows of the table, all T output rows, the ids."""
    ids = np.asarray(ids)
    T, rows = ids.size, np.unique(ids).size
    row_bytes = 4 * D if qtype is None else -(-D // 32) * BLOCK_BYTES[qtype]
    return rows * row_bytes + 4 * T * D + 4 * T


def bytes_chain(cfg, T, with_gather=True):
    b = (bytes_add_rmsnorm(T, cfg["dim"]) + bytes_rope(T, cfg["n_heads"], cfg["n_kv_heads"],
                                                        cfg["head_dim"])
         + bytes_swiglu(T, cfg["ffn"]))
    if with_gather:
        b += bytes_gather_f32(T, cfg["dim"])
    return b


# ------------------------------------------------------- linear layers
# The seven projections of one Llama layer, (name, in_features,
# out_features): wq, wk, wv, wo, w_gate, w_up, w_down.

def layer_linears(cfg):
    D, H, KV, hd, F = cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["ffn"]
    return (("wq", D, H * hd), ("wk", D, KV * hd), ("wv", D, KV * hd), ("wo", H * hd, D),
            ("w_gate", D, F), ("w_up", D, F), ("w_down", F, D))


def weight_bytes(qtype, in_features, out_features):
    """Bytes of one weight matrix: fp32 [out, in], or out rows of
    ceil(in / 32) blocks."""
    if qtype == "f32":
        return 4 * in_features * out_features
    return out_features * -(-in_features // 32) * BLOCK_BYTES[qtype]


def bytes_linear(qtype, T, in_features, out_features):
    """Read the weight once, read x [T, in], write y [T, out]."""
    return weight_bytes(qtype, in_features, out_features) + 4 * T * (in_features + out_features)


def flops_linear(T, in_features, out_features):
    return 2 * T * in_features * out_features


# ------------------------------------------------------- decode attention

def flops_prefill_attention(T, H, hd, pos0=0):
    """Causal attention of T tokens at positions pos0 + t: per head and
    attended position, q.k and p v, 2 hd flops each."""
    n_pairs = T * pos0 + T * (T + 1) // 2
    return 4 * hd * H * n_pairs


def flops_decode_attention(positions, n_heads, head_dim):
    """Decode tokens at the given positions: per head and attended position
    (0..pos), q.k and p v, 2 hd flops each."""
    pos = np.asarray(positions, np.int64)
    return int(4 * head_dim * n_heads * (pos + 1).sum())


def bytes_attention(positions, n_heads, n_kv_heads, head_dim):
    """Read the K and V rows 0..pos of each token's KV heads once, read q,
    write out: 8 * (pos + 1) * KV * hd per token + 8 * H * hd."""
    pos = np.asarray(positions, np.int64)
    return int(8 * (pos + 1).sum() * n_kv_heads * head_dim + 8 * pos.size * n_heads * head_dim)
