"""CPU tests that pin the oracle (oracle/oracle.c) before anything trusts it.

1. The oracle passes every pin (reference known answers, closed forms,
   invariants) in tests/pins.py.
2. Planted mistakes — each a plausible bug in a restatement — fail at least
   one pin, so passing the pins means something.
3. Cross-checks against independent float64 computations (math.fsum, numpy,
   torch CPU SDPA) on random inputs.
4. The seeded generator and the fp16 rounding are pinned exhaustively or
   statistically.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
import pins

# ------------------------------------------------------------------ oracle passes


def test_pin_reduce():
    pins.pin_reduce(oracle.reduce_sum)


def test_pin_softmax():
    pins.pin_softmax(oracle.softmax)


def test_pin_transpose():
    pins.pin_transpose(oracle.transpose)


def test_pin_rmsnorm():
    pins.pin_rmsnorm(oracle.rmsnorm)


def test_pin_gemm():
    pins.pin_gemm(oracle.gemm)


def test_pin_attention():
    pins.pin_attention(oracle.attention)


# --------------------------------------------------------- planted mistakes fail


def _fails(pin, f):
    with pytest.raises(AssertionError):
        pin(f)


def test_planted_reduce_mistakes():
    _fails(pins.pin_reduce, lambda x: oracle.reduce_sum(x[1:]))          # dropped term
    _fails(pins.pin_reduce, lambda x: float(np.float32(x).sum(dtype=np.float32))
           if x.size > 50_000 else oracle.reduce_sum(x) + 0.5)        # biased / fp32 sum
    _fails(pins.pin_reduce, lambda x: abs(oracle.reduce_sum(x)))        # sign


def test_planted_softmax_mistakes():
    def no_max_shift(x):
        x = x.astype(np.float32)
        with np.errstate(over="ignore", invalid="ignore"):
            e = np.exp(x.astype(np.float32)).astype(np.float64)
            return e / e.sum(-1, keepdims=True)

    def unnormalised(x):
        return oracle.softmax(x) * 1.5

    def wrong_axis(x):
        y = np.exp(x.astype(np.float64) - x.max(0, keepdims=True))
        return y / y.sum(0, keepdims=True)

    def negated(x):
        return oracle.softmax(-x)

    for f in (no_max_shift, unnormalised, wrong_axis, negated):
        _fails(pins.pin_softmax, f)


def test_planted_transpose_mistakes():
    _fails(pins.pin_transpose, lambda x: x.reshape(x.shape[1], x.shape[0]).copy())
    _fails(pins.pin_transpose, lambda x: np.flip(oracle.transpose(x), 0).copy())


def test_planted_rmsnorm_mistakes():
    def no_eps(x, w, eps):
        return oracle.rmsnorm(x, w, 1e-38)

    def mean_over_h_minus_1(x, w, eps):
        x64 = x.astype(np.float64)
        ms = (x64 ** 2).sum(-1, keepdims=True) / (x.shape[-1] - 1)
        return x64 / np.sqrt(ms + eps) * w

    def no_weight(x, w, eps):
        return oracle.rmsnorm(x, np.ones_like(w), eps)

    for f in (no_eps, mean_over_h_minus_1, no_weight):
        _fails(pins.pin_rmsnorm, f)


def test_planted_gemm_mistakes():
    def transposed_b(a, b):
        return oracle.gemm(a, np.ascontiguousarray(b.T)) if b.shape[0] == b.shape[1] \
            else oracle.gemm(a, np.ascontiguousarray(b.T.reshape(b.shape)))

    def dropped_last_k(a, b):
        return oracle.gemm(np.ascontiguousarray(a[:, :-1]), np.ascontiguousarray(b[:-1]))

    for f in (transposed_b, dropped_last_k):
        _fails(pins.pin_gemm, f)


def _numpy_attention(q, k, v, causal, scale_pow=0.5, mask_offset=0, swap_kv=False):
    """Independent float64 attention used only for the planted-mistake tests."""
    q, k, v = (t.astype(np.float64) for t in (q, k, v))
    if swap_kv:
        k, v = v, k
    d = q.shape[-1]
    s = q @ np.swapaxes(k, -1, -2) / d ** scale_pow
    if causal:
        n = s.shape[-1]
        hide = np.arange(n)[None, :] > np.arange(n)[:, None] + mask_offset
        s = np.where(hide, -np.inf, s)
    with np.errstate(invalid="ignore"):
        p = np.exp(s - s.max(-1, keepdims=True))
        return (p / p.sum(-1, keepdims=True)) @ v


def test_planted_attention_mistakes():
    pins.pin_attention(_numpy_attention)  # the independent version passes
    mistakes = [
        lambda q, k, v, c: _numpy_attention(q, k, v, c, scale_pow=1.0),    # 1/D scale
        lambda q, k, v, c: _numpy_attention(q, k, v, c, mask_offset=-1),   # j < i
        lambda q, k, v, c: _numpy_attention(q, k, v, c, mask_offset=1),    # j <= i+1
        lambda q, k, v, c: _numpy_attention(q, k, v, c, swap_kv=True),     # K <-> V
        lambda q, k, v, c: _numpy_attention(q, k, v, False),               # mask dropped
    ]
    for f in mistakes:
        _fails(pins.pin_attention, f)


# -------------------------------------------------------- independent cross-checks


def test_reduce_matches_fsum():
    x = oracle.uniform(21, 1 << 20)
    assert oracle.reduce_sum(x) == pytest.approx(math.fsum(x.astype(np.float64)),
                                                 rel=0, abs=1e-9)


def test_softmax_matches_numpy():
    x = oracle.normal(22, (33, 257), 0.0, 3.0)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(-1, keepdims=True))
    np.testing.assert_allclose(oracle.softmax(x), e / e.sum(-1, keepdims=True),
                               rtol=1e-6, atol=0)


def test_rmsnorm_matches_numpy():
    x = oracle.normal(23, (17, 1003))
    w = oracle.uniform(24, 1003, 0.5, 1.5)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + np.float64(np.float32(1e-6))) * w
    np.testing.assert_allclose(oracle.rmsnorm(x, w, 1e-6), ref, rtol=1e-13, atol=1e-15)


def test_gemm_matches_numpy_and_row_subset():
    a = oracle.uniform(25, (37, 71))
    b = oracle.uniform(26, (71, 65))
    full = oracle.gemm(a, b)
    np.testing.assert_allclose(full, a.astype(np.float64) @ b.astype(np.float64),
                               rtol=1e-13, atol=1e-13)
    rows = [36, 0, 5]
    np.testing.assert_array_equal(oracle.gemm(a, b, rows), full[rows])


def test_attention_matches_torch_sdpa_and_row_subset():
    torch = pytest.importorskip("torch")
    q = oracle.normal(27, (1, 2, 37, 71))
    k = oracle.normal(28, (1, 2, 37, 71))
    v = oracle.normal(29, (1, 2, 37, 71))
    for causal in (False, True):
        ref = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q).double(), torch.from_numpy(k).double(),
            torch.from_numpy(v).double(), is_causal=causal).numpy()
        full = oracle.attention(q, k, v, causal)
        np.testing.assert_allclose(full, ref, rtol=1e-11, atol=1e-12)
        heads, rows = [1, 0, 1], [36, 0, 17]
        sub = oracle.attention(q, k, v, causal, heads, rows)
        np.testing.assert_array_equal(sub, full.reshape(2, 37, 71)[heads, rows])


# ------------------------------------------------------------ generator and fp16


def test_f16_conversion_exhaustive():
    bits = np.arange(1 << 16, dtype=np.uint16)
    as_f32 = bits.view(np.float16).astype(np.float32)
    got = oracle.from_f16_bits(bits)
    finite = np.isfinite(as_f32)
    assert np.array_equal(got[finite].view(np.uint32), as_f32[finite].view(np.uint32))
    assert np.all(np.isnan(got[~np.isfinite(as_f32) & np.isnan(as_f32)]))
    # round trip of every finite half, and RNE on random fp32 values vs numpy
    back = oracle.to_f16_bits(got[finite])
    assert np.array_equal(back, bits[finite])
    x = np.concatenate([oracle.normal(30, 200_000, 0.0, 4.0),
                        oracle.uniform(31, 100_000, -70000.0, 70000.0),
                        oracle.normal(32, 100_000, 0.0, 1e-5)])
    with np.errstate(over="ignore"):
        assert np.array_equal(oracle.to_f16_bits(x), x.astype(np.float16).view(np.uint16))


def test_generator_is_deterministic_and_in_range():
    a = oracle.uniform(123, 100_000)
    assert np.array_equal(a, oracle.uniform(123, 100_000))
    assert not np.array_equal(a, oracle.uniform(124, 100_000))
    assert a.min() >= -1.0 and a.max() < 1.0
    assert abs(a.mean()) < 0.01 and abs(a.var() - 1.0 / 3.0) < 0.01
    # every value is -1 + j * 2^-23 exactly (24-bit mapping)
    assert np.all(((a.astype(np.float64) + 1.0) * 2 ** 23) % 1 == 0)
    z = oracle.normal(5, 400_000, 0.0, 3.0)
    assert abs(z.mean()) < 0.03 and abs(z.std() - 3.0) < 0.03
    # SplitMix64 known answer (first output for seed 0 per its published
    # reference implementation)
    assert oracle.uniform(0, 1)[0] == np.float32(-1.0 + 2.0 * (0xE220A8397B1DCDAF >> 40) / 2 ** 24)
