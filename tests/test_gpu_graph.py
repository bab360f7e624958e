"""HIP-graph capture of an op chain: every replay must equal the eager run.

The chain is the decode step of configs[1] (gather -> add + RMSNorm ->
RoPE -> SwiGLU, T = 4).  The graph is replayed several times with eager work
(re-uploading the in-place RoPE inputs) and device synchronizations between
the replays, and each replay is compared with the eager result bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_bits_equal, load_workloads

W = load_workloads()
pytestmark = pytest.mark.gpu


def test_graph_replays_equal_eager(mlk):
    cfg = W.CONFIGS["c2_decode_8b"]
    T, V, D, H, KV, hd, F = 4, 4096, cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], \
        cfg["head_dim"], cfg["ffn"]
    rng = np.random.default_rng(5)
    table = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    ids = np.array([3, 4095, 0, 17], np.int32)
    pos = np.array([8191, 0, 4095, 12], np.int32)
    delta = (rng.standard_normal((T, D)) * 0.02).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    q = (rng.standard_normal((T, H * hd)) * 0.02).astype(np.float32)
    k = (rng.standard_normal((T, KV * hd)) * 0.02).astype(np.float32)
    gate = rng.standard_normal((T, F)).astype(np.float32)
    up = rng.standard_normal((T, F)).astype(np.float32)
    d = {n: mlk.DeviceBuffer.from_array(a) for n, a in dict(
        table=table, ids=ids, pos=pos, delta=delta, w=w, q=q, k=k, gate=gate, up=up).items()}
    d["x"] = mlk.DeviceBuffer.empty((T, D))
    d["y"] = mlk.DeviceBuffer.empty((T, D))
    d["o"] = mlk.DeviceBuffer.empty((T, F))
    stream = mlk.Stream()

    def chain():
        mlk.gather_f32(d["table"], V, D, d["ids"], T, d["x"], stream=stream)
        mlk.add_rmsnorm(d["x"], d["delta"], d["w"], d["y"], T, D, cfg["eps"], stream=stream)
        mlk.rope(d["q"], d["k"], T, H, KV, hd, positions=d["pos"], theta=cfg["theta"],
                 stream=stream)
        mlk.swiglu(d["gate"], d["up"], d["o"], T * F, stream=stream)

    def outputs():
        stream.synchronize()
        return [d[n].download() for n in ("x", "y", "q", "k", "o")]

    chain()
    eager = outputs()
    d["q"].upload(q)
    d["k"].upload(k)
    with mlk.Graph.capture(stream) as graph:
        chain()
    for replay in range(4):
        # eager work between replays: reset the in-place RoPE inputs and
        # scribble over the outputs, then synchronize
        d["q"].upload(q)
        d["k"].upload(k)
        d["y"].zero(stream)
        d["o"].zero(stream)
        mlk.synchronize()
        graph.launch()
        for got, want, name in zip(outputs(), eager, ("x", "y", "q", "k", "o")):
            assert_bits_equal(got, want, f"replay {replay} {name}")
    graph.close()


def test_null_stream_cannot_be_captured(mlk):
    with pytest.raises(mlk.MlkError, match="null stream"):
        with mlk.Graph.capture(None):
            pass
