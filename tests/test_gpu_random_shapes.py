"""Seeded random shapes and misaligned bases, every operator against the oracle.

The shape-specific tests pin the dispatch boundaries the kernels were written
around; this module draws shapes the code was not written for: sizes near 1,
near tile multiples (28..70, 120..140, 250..270, 500..530, 1000..1030) and
past them, head dims of any value up to 128, ragged sequence lengths, and
base pointers 0..3 elements past an allocation's start. Each case is seeded
(operator, index), so a failure names a reproducible input. Tolerances are
the library's accuracy contract: transpose bit-exact; reduce,
softmax and RMSNorm relative 1e-5 (softmax absolute 1e-6 on probabilities);
fp32 GEMM Frobenius 1e-4 over the checked rows; fp16 GEMM and fp16
attention max-abs 2e-3; fp32 attention 1e-4 + 1e-4 |ref|.
"""

from __future__ import annotations

import zlib

import numpy as np
import pytest

import oracle
from gpu_util import HipOps

pytestmark = pytest.mark.gpu

CASES = 24  # per operator

_BANDS = ((1, 20), (28, 70), (120, 140), (250, 270), (500, 530), (1000, 1030))


@pytest.fixture(scope="module")
def hip(lib):
    return HipOps(lib)


def _rng(op: str, i: int) -> np.random.Generator:
    return np.random.default_rng(zlib.crc32(f"{op}/{i}".encode()))


def _dim(rng: np.random.Generator) -> int:
    lo, hi = _BANDS[rng.integers(len(_BANDS))]
    return int(rng.integers(lo, hi + 1))


def _seed(rng: np.random.Generator) -> int:
    return int(rng.integers(1 << 30))


@pytest.mark.parametrize("i", range(CASES))
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_random_gemm(hip, dtype, i):
    rng = _rng(f"gemm_{dtype}", i)
    m, n, k = _dim(rng), _dim(rng), _dim(rng)
    if i % 4 == 3:  # a larger product, rows sampled
        m, n, k = (int(rng.integers(1500, 2600)) for _ in range(3))
    off, s = int(rng.integers(0, 4)), _seed(rng)
    a, b = oracle.uniform(s, (m, k)), oracle.uniform(s + 1, (k, n))
    rows = np.unique(np.concatenate([[0, m - 1], rng.integers(0, m, 48)])).astype(np.int32)
    if dtype == "f16":
        ab, bb = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(ab, bb, off)
        ref = oracle.gemm(oracle.from_f16_bits(ab), oracle.from_f16_bits(bb), rows)
        assert np.max(np.abs(y[rows] - ref)) <= 2e-3, (m, n, k, off)
    else:
        y = hip.gemm_f32(a, b, off)
        ref = oracle.gemm(a, b, rows)
        assert np.linalg.norm(y[rows] - ref) <= 1e-4 * np.linalg.norm(ref), (m, n, k, off)
    assert np.isfinite(y).all()


@pytest.mark.parametrize("i", range(CASES))
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_random_attention(hip, dtype, i):
    rng = _rng(f"attention_{dtype}", i)
    b, h = int(rng.integers(1, 3)), int(rng.integers(1, 6))
    s = int(rng.choice([rng.integers(1, 70), rng.integers(100, 700), rng.integers(700, 1300)]))
    d = int(rng.choice([16, 32, 48, 64, 64, 80, 96, 128, 128, int(rng.integers(1, 129))]))
    causal = bool(rng.integers(2))
    off, seed = int(rng.integers(0, 4)), _seed(rng)
    q, k, v = (oracle.normal(seed + j, (b, h, s, d)) for j in range(3))
    heads = np.repeat(np.arange(b * h, dtype=np.int32), 12)
    rows = rng.integers(0, s, heads.size).astype(np.int32)
    if dtype == "f16":
        qb, kb, vb = (oracle.to_f16_bits(t) for t in (q, k, v))
        y = hip.attention(qb, kb, vb, causal, off)
        ref = oracle.attention(*(oracle.from_f16_bits(t) for t in (qb, kb, vb)), causal,
                               heads, rows)
        got = y.reshape(b * h, s, d)[heads, rows]
        assert np.max(np.abs(got - ref)) <= 2e-3, (b, h, s, d, causal, off)
    else:
        y = hip.attention(q, k, v, causal, off)
        ref = oracle.attention(q, k, v, causal, heads, rows)
        got = y.reshape(b * h, s, d)[heads, rows]
        assert np.all(np.abs(got - ref) <= 1e-4 + 1e-4 * np.abs(ref)), (b, h, s, d, causal, off)
    assert np.isfinite(y).all()


@pytest.mark.parametrize("i", range(CASES))
def test_random_transpose(hip, i):
    rng = _rng("transpose", i)
    r, c = int(rng.integers(1, 3000)), int(rng.integers(1, 3000))
    if i % 3 == 2:  # multiples of 4: the float4 kernels
        r, c = 4 * int(rng.integers(1, 800)), 4 * int(rng.integers(1, 800))
    off, s = int(rng.integers(0, 4)), _seed(rng)
    x = oracle.uniform(s, (r, c))
    y = hip.transpose(x, off)
    assert y.view(np.uint32).tobytes() == oracle.transpose(x).view(np.uint32).tobytes(), (r, c, off)


@pytest.mark.parametrize("i", range(CASES))
def test_random_softmax(hip, i):
    rng = _rng("softmax", i)
    r, c = int(rng.integers(1, 3000)), int(rng.integers(1, 9000))
    off, s = int(rng.integers(0, 4)), _seed(rng)
    x = oracle.normal(s, (r, c), 0.0, 3.0)
    assert np.max(np.abs(hip.softmax(x, off) - oracle.softmax(x))) <= 1e-6, (r, c, off)


@pytest.mark.parametrize("i", range(CASES))
def test_random_rmsnorm(hip, i):
    rng = _rng("rmsnorm", i)
    r, c = int(rng.integers(1, 3000)), int(rng.integers(1, 9000))
    off, s = int(rng.integers(0, 4)), _seed(rng)
    x = oracle.normal(s, (r, c))
    w = oracle.uniform(s + 1, c, 0.5, 1.5)
    ref = oracle.rmsnorm(x, w, 1e-6)
    y = hip.rmsnorm(x, w, 1e-6, off)
    assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), 1e-3)) <= 1e-5, (r, c, off)


@pytest.mark.parametrize("i", range(CASES))
def test_random_reduce(hip, i):
    rng = _rng("reduce", i)
    n = int(rng.integers(1, 5000)) if i % 2 else int(rng.integers(5000, 5_000_000))
    off, s = int(rng.integers(0, 4)), _seed(rng)
    x = oracle.uniform(s, n)
    ref = oracle.reduce_sum(x)
    assert abs(hip.reduce_sum(x, off) - ref) <= 1e-5 * max(abs(ref), 1.0), (n, off)
