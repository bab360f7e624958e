"""The bf16 piece split the matrix-core kernels use, checked on the CPU.

A float x is split into three bf16 values: hi = x with its low 16 bits
cleared, mid = the same of x - hi, lo = (x - hi) - mid.  The kernels rely on
three facts, pinned here by direct computation in float64 (every product of
two bf16 values, and every sum of a few of them, is exact there):
  - hi + mid + lo == x exactly (so a small integer code times the three
    pieces, the linear layers' products, is code * x exactly);
  - |mid| < 2^-7 |x| and |lo| < 2^-14 |x|, lo with at most 8 significant bits;
  - keeping the six products a_i b_j with i + j <= 2 (0 = hi, 1 = mid,
    2 = lo) of the nine, as the attention tiles' scores and values do, leaves
    an error below 2^-20 |a b| (16 u).
"""
from __future__ import annotations

import numpy as np

TOP16 = np.uint32(0xFFFF0000)


def split3(x):
    """(hi, mid, lo) of float32 x as float32 arrays (the kernels' SplitBf for
    finite values: mask, subtract, mask, subtract)."""
    x = np.asarray(x, np.float32)
    hi = (x.view(np.uint32) & TOP16).view(np.float32)
    r = (x - hi).astype(np.float32)
    mid = (r.view(np.uint32) & TOP16).view(np.float32)
    lo = (r - mid).astype(np.float32)
    return hi, mid, lo


def samples(rng, n):
    """Random normals over a wide exponent range, values with every
    significand bit set, powers of two and the smallest normal."""
    a = rng.standard_normal(n) * np.exp2(rng.integers(-60, 60, n))
    full = np.ldexp(2.0 - 2.0 ** -23, rng.integers(-60, 60, n)) * np.where(rng.random(n) < 0.5, -1, 1)
    edge = np.array([1.0, -1.0, 2.0 ** -126, 3.0, 1.0 + 2.0 ** -23, 65504.0])
    return np.concatenate([a, full, edge]).astype(np.float32)


def test_split_is_exact_and_pieces_are_small():
    x = samples(np.random.default_rng(1), 20000)
    hi, mid, lo = split3(x)
    x64 = x.astype(np.float64)
    assert np.array_equal(hi.astype(np.float64) + mid.astype(np.float64) + lo.astype(np.float64), x64)
    ax = np.abs(x64)
    assert (np.abs(mid.astype(np.float64)) < 2.0 ** -7 * ax).all()
    assert (np.abs(lo.astype(np.float64)) < 2.0 ** -14 * ax).all()
    # every piece is a bf16 value: its low 16 bits are zero
    for p in (hi, mid, lo):
        assert not (p.view(np.uint32) & np.uint32(0xFFFF)).any()


def test_code_times_pieces_is_exact():
    rng = np.random.default_rng(2)
    x = samples(rng, 5000)
    code = rng.integers(-128, 128, x.size).astype(np.float64)
    hi, mid, lo = (p.astype(np.float64) for p in split3(x))
    assert np.array_equal(code * hi + code * mid + code * lo, code * x.astype(np.float64))


def test_six_of_nine_products_within_2_pow_minus_20():
    rng = np.random.default_rng(3)
    a, b = samples(rng, 20000), samples(rng, 20000)
    # keep the products in range of float64 without underflow
    a = np.ldexp(np.frexp(a)[0], rng.integers(-20, 20, a.size)).astype(np.float32)
    b = np.ldexp(np.frexp(b)[0], rng.integers(-20, 20, b.size)).astype(np.float32)
    pa = [p.astype(np.float64) for p in split3(a)]
    pb = [p.astype(np.float64) for p in split3(b)]
    kept = sum(pa[i] * pb[j] for i in range(3) for j in range(3) if i + j <= 2)
    exact = a.astype(np.float64) * b.astype(np.float64)
    err = np.abs(kept - exact)
    assert (err <= 2.0 ** -20 * np.abs(exact)).all()
    # and the bound is near tight for full significands (it is not loose by a
    # large factor, so the tests' 16 u a product is the right term)
    worst = float((err / np.maximum(np.abs(exact), 1e-300)).max())
    assert worst > 2.0 ** -22
