"""Known-answer checks ("pins") for each operator.

Every pin takes an implementation with the oracle's calling convention
(numpy in, numpy out) and raises AssertionError when it disagrees with a
value fixed by the reference's own known-answer tests, by a closed form, or
by an invariant. They are chosen so that the plausible mistakes — a dropped
term (eps, the max shift, the normalisation), a wrong sign or index, a
transposed operand, an off-by-one causal mask, a wrong softmax scale — each
fail at least one pin; tests/test_oracle.py demonstrates that on planted
mistakes. The same pins run against the GPU kernels in the GPU tests, with
tolerances suited to fp32/fp16 arithmetic.
"""

from __future__ import annotations

import math

import numpy as np

# --------------------------------------------------------------------- reduce


def pin_reduce(f, tol_rel: float = 0.0) -> None:
    # tests/core_ops_smoke.cu:33-36: iota -500..499 sums to exactly -500.
    x = np.arange(-500, 500, dtype=np.float32)
    assert f(x) == -500.0
    # all ones -> N (exact in fp32 while N < 2^24)
    n = 1_000_003
    assert abs(f(np.ones(n, np.float32)) - n) <= tol_rel * n
    # sign: all -0.5 -> -N/2
    assert abs(f(np.full(4096, -0.5, np.float32)) + 2048.0) <= tol_rel * 2048
    # independent exactly-rounded sum (math.fsum) of a zero-mean input
    rng = np.random.default_rng(7)
    x = rng.uniform(-1, 1, 100_000).astype(np.float32)
    exact = math.fsum(x.astype(np.float64))
    bound = max(tol_rel * abs(exact), 1e-9 * float(np.abs(x).sum()))
    assert abs(f(x) - exact) <= bound, (f(x), exact)


# -------------------------------------------------------------------- softmax


def pin_softmax(f, tol: float = 1e-12) -> None:
    # two-element closed form
    a, b = 0.75, -1.25
    y = f(np.array([[a, b]], np.float32))
    assert abs(y[0, 0] - 1.0 / (1.0 + math.exp(b - a))) <= tol
    assert abs(y[0, 1] - 1.0 / (1.0 + math.exp(a - b))) <= tol
    # constant row -> 1/cols
    y = f(np.full((3, 7), 2.5, np.float32))
    assert np.all(np.abs(y - 1.0 / 7.0) <= tol)
    # one-hot at +-1000 (needs the max shift): exactly [0..1..0]
    x = np.full((2, 9), -1000.0, np.float32)
    x[0, 4] = 1000.0
    x[1, 0] = 1000.0
    y = f(x)
    expect = np.zeros_like(y)
    expect[0, 4] = 1.0
    expect[1, 0] = 1.0
    assert np.all(np.abs(y - expect) <= tol)
    # rows sum to 1; shift invariance (shift exact in fp32)
    rng = np.random.default_rng(11)
    x = (rng.integers(-64, 64, (5, 33)) / 8.0).astype(np.float32)
    y = f(x)
    assert np.all(np.abs(y.sum(-1) - 1.0) <= 64 * tol)
    assert np.all(np.abs(f(x + np.float32(3.0)) - y) <= tol)
    # ordering follows the input ordering
    assert np.all(np.argsort(y[0], kind="stable") == np.argsort(x[0], kind="stable"))


# ------------------------------------------------------------------ transpose


def pin_transpose(f) -> None:
    # tests/core_ops_smoke.cu:94-119: 37x65 iota, value encodes the index
    rows, cols = 37, 65
    x = (np.arange(rows * cols, dtype=np.float32) - 100.0).reshape(rows, cols)
    y = f(x)
    assert y.shape == (cols, rows)
    r, c = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    assert np.array_equal(y[c, r], x[r, c])
    assert np.array_equal(y[c, r], (r * cols + c - 100).astype(np.float32))
    # involution on an odd, non-square shape
    x = np.random.default_rng(3).standard_normal((13, 70)).astype(np.float32)
    assert np.array_equal(f(f(x)), x)


# -------------------------------------------------------------------- rmsnorm


def pin_rmsnorm(f, tol: float = 1e-12) -> None:
    # constant row c: y = c / sqrt(c^2 + eps) * w
    c, eps, h = 1.5, 0.25, 6
    w = np.linspace(0.5, 1.5, h).astype(np.float32)
    y = f(np.full((2, h), c, np.float32), w, eps)
    expect = c / math.sqrt(c * c + eps) * w.astype(np.float64)
    assert np.all(np.abs(y - expect) <= tol * 4)
    # [3, 4] with eps 0.5: mean square 12.5 -> inv = 1/sqrt(13)
    y = f(np.array([[3.0, 4.0]], np.float32), np.array([1.0, 2.0], np.float32), 0.5)
    assert abs(y[0, 0] - 3.0 / math.sqrt(13.0)) <= tol * 4
    assert abs(y[0, 1] - 8.0 / math.sqrt(13.0)) <= tol * 4
    # zero row -> zeros (eps keeps it finite)
    y = f(np.zeros((1, 5), np.float32), np.ones(5, np.float32), 1e-6)
    assert np.all(y == 0.0)
    # weight linearity and unit RMS with w = 1, tiny eps
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 100)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 100).astype(np.float32)
    y1 = f(x, w, 1e-6)
    y2 = f(x, (2 * w).astype(np.float32), 1e-6)
    assert np.all(np.abs(y2 - 2 * y1) <= tol * 16)
    y = f(x, np.ones(100, np.float32), 1e-30)
    assert np.all(np.abs(np.sqrt((y.astype(np.float64) ** 2).mean(-1)) - 1.0) <= tol * 64)


# ----------------------------------------------------------------------- gemm


def pin_gemm(f, tol: float = 0.0) -> None:
    rng = np.random.default_rng(9)
    # rectangular small-integer product: exact, catches transposed operands
    a = rng.integers(-4, 5, (7, 5)).astype(np.float32)
    b = rng.integers(-4, 5, (5, 3)).astype(np.float32)
    expect = a.astype(np.int64) @ b.astype(np.int64)
    assert np.all(np.abs(f(a, b) - expect) <= tol * np.abs(expect).max())
    # identity and permutation (entries k/8: exact in fp16 and fp32)
    m = (rng.integers(-64, 64, (6, 6)) / 8.0).astype(np.float32)
    assert np.all(np.abs(f(m, np.eye(6, dtype=np.float32)) - m) <= tol)
    perm = rng.permutation(6)
    p = np.eye(6, dtype=np.float32)[perm]
    assert np.all(np.abs(f(p, m) - m[perm]) <= tol)
    # rank one u v^T
    u = np.array([[1.0], [-2.0], [0.5]], np.float32)
    v = np.array([[4.0, -1.0, 0.25, 3.0]], np.float32)
    assert np.all(np.abs(f(u, v) - u.astype(np.float64) @ v.astype(np.float64)) <= tol)


# ------------------------------------------------------------------ attention


def pin_attention(f, tol: float = 1e-12) -> None:
    """f(q, k, v, causal) on [B, H, S, D] float32 arrays -> [B, H, S, D]."""
    rng = np.random.default_rng(13)
    b, h, s, d = 1, 2, 9, 8
    q = rng.standard_normal((b, h, s, d)).astype(np.float32)
    k = rng.standard_normal((b, h, s, d)).astype(np.float32)
    # V identical for every key -> O equals that row, causal or not
    vrow = rng.standard_normal(d).astype(np.float32)
    v = np.broadcast_to(vrow, (b, h, s, d)).copy()
    for causal in (False, True):
        assert np.all(np.abs(f(q, k, v, causal) - vrow) <= tol)
    # all keys equal -> uniform weights: global mean / causal prefix mean
    v = rng.standard_normal((b, h, s, d)).astype(np.float32)
    keq = np.broadcast_to(k[:, :, :1, :], k.shape).copy()
    o = f(q, keq, v, False)
    assert np.all(np.abs(o - v.astype(np.float64).mean(2, keepdims=True)) <= tol)
    o = f(q, keq, v, True)
    prefix = np.cumsum(v.astype(np.float64), axis=2) / np.arange(1, s + 1)[:, None]
    assert np.all(np.abs(o - prefix) <= tol)
    # causal row 0 sees only key 0; last row sees everything
    oc = f(q, k, v, True)
    on = f(q, k, v, False)
    assert np.all(np.abs(oc[:, :, 0, :] - v[:, :, 0, :]) <= tol)
    assert np.all(np.abs(oc[:, :, -1, :] - on[:, :, -1, :]) <= tol)
    # two keys, D = 4: weights softmax(q.k_j / sqrt(4)) by hand
    q2 = np.array([[[[0.5, -1.0, 2.0, 0.25]] * 2]], np.float32)
    k2 = np.array([[[[1.0, 0.5, -0.5, 2.0], [-1.0, -1.5, 0.75, 1.0]]]], np.float32)
    v2 = np.array([[[[1.0, 2.0, 3.0, 4.0], [-2.0, 0.0, 1.0, 5.0]]]], np.float32)
    s0 = float(q2[0, 0, 0] @ k2[0, 0, 0]) / 2.0
    s1 = float(q2[0, 0, 0] @ k2[0, 0, 1]) / 2.0
    w0 = 1.0 / (1.0 + math.exp(s1 - s0))
    v64 = v2.astype(np.float64)
    expect = w0 * v64[0, 0, 0] + (1.0 - w0) * v64[0, 0, 1]
    o = f(q2, k2, v2, False)
    assert np.all(np.abs(o[0, 0, 0] - expect) <= tol)
    assert np.all(np.abs(f(q2, k2, v2, True)[0, 0, 0] - v2[0, 0, 0]) <= tol)
