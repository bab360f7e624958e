"""The no-allocation decode attention entry (mlk_attention_decode_f32_noalloc)
against the entry it varies (mlk_attention_decode_f32 with a caller
workspace), through the C ABI.

Both run the same kernels on the same chunk plan, so the outputs must be
equal bit for bit.  Two calls in a row go through the library's fixed
scratch, the second with a smaller input (fewer tokens, a shorter context,
another kernel path), so stale partials of the first call would show in the
second.  The shapes need chunk partials (the scratch is really used): the
8B head layout (32 query / 8 KV heads, head_dim 128) at positions up to 8191.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

L, S, KV, HD, H = 2, 8192, 8, 128, 32


@pytest.fixture(scope="module")
def cache(mlk):
    rng = np.random.default_rng(1234)
    kc = (rng.standard_normal((L, S, KV, HD)) * 0.5).astype(np.float32)
    vc = rng.standard_normal((L, S, KV, HD)).astype(np.float32)
    return mlk.DeviceBuffer.from_array(kc), mlk.DeviceBuffer.from_array(vc)


def run_both(mlk, cache, T, max_ctx, positions, seed):
    k, v = cache
    rng = np.random.default_rng(seed)
    q = mlk.DeviceBuffer.from_array(rng.standard_normal((T, H, HD)).astype(np.float32))
    pos = mlk.DeviceBuffer.from_array(np.asarray(positions, np.int32))
    need = mlk.attention_workspace_bytes(T, H, KV, HD, max_ctx)
    assert 0 < need <= mlk.attention_noalloc_scratch_bytes()
    ws = mlk.DeviceBuffer(need, np.uint8)
    want = mlk.DeviceBuffer.empty((T, H, HD))
    got = mlk.DeviceBuffer.empty((T, H, HD))
    print(f"no-alloc attention: T={T} max_ctx={max_ctx} partials={need} B", flush=True)
    mlk.attention_decode(q, k, v, L, S, H, KV, HD, 1, T, want, max_ctx, positions=pos,
                         workspace=ws, workspace_bytes=need)
    mlk.attention_decode_noalloc(q, k, v, L, S, H, KV, HD, 1, T, got, max_ctx, positions=pos)
    mlk.synchronize()
    a, b = want.download(), got.download()
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
        f"T={T}: {int((a != b).sum())} elements differ"


def test_noalloc_matches_workspace_entry_twice(mlk, cache):
    rng = np.random.default_rng(7)
    # first: 16 tokens at positions across the whole context (shared-tile path)
    run_both(mlk, cache, 16, S, rng.integers(0, S, 16), seed=1)
    # second, smaller: one token on a shorter context (per-token path)
    run_both(mlk, cache, 1, 4096, [3001], seed=2)


def test_noalloc_rejects_more_than_the_scratch(mlk):
    limit = mlk.attention_noalloc_scratch_bytes()
    assert limit == 64 << 20
    T, max_ctx = 1024, 1 << 17
    assert mlk.attention_workspace_bytes(T, 64, 8, 128, max_ctx) > limit
    # null operands: the size check comes first and names the scratch; were it
    # ever moved after the operand checks, those would reject the nulls with
    # another message (a clean failure here, never a launch)
    with pytest.raises(mlk.MlkError, match="exceed the .*-byte scratch"):
        mlk.attention_decode_noalloc(None, None, None, 1, max_ctx, 64, 8, 128, 0, T,
                                     None, max_ctx, pos0=0)
