"""Inputs past 2^31 elements: every launcher indexes with 64-bit offsets.

Each case builds a device tensor of slightly more than 2^31 elements (8-9 GB
in fp32) on the GPU, runs the operator through the C ABI and checks it
against the CPU oracle on seeded row samples that always include the first
and last rows, where a 32-bit index would wrap. Reduce sums ones, so a
dropped or repeated element changes the exactly known result.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from gpu_util import check, ptr, stream_handle

pytestmark = pytest.mark.gpu

BIG = 2 ** 31


def _randn(shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, generator=g, device="cuda") * scale).to(dtype)


def _rows(n: int, seed: int, count: int = 24) -> np.ndarray:
    rng = np.random.default_rng(seed)
    r = set(rng.integers(0, n, count).tolist()) | {0, 1, n - 2, n - 1}
    return np.array(sorted(r), dtype=np.int64)


@pytest.fixture(autouse=True)
def _free_memory():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def test_reduce_past_2g_elements(lib):
    n = BIG + 13
    x = torch.ones(n, device="cuda")
    out = torch.empty(1, device="cuda")
    check(lib.operatorlib_reduce_sum_f32(ptr(x), ptr(out), n, stream_handle()), "reduce")
    torch.cuda.synchronize()
    # fp64 accumulation: exactly n, then one rounding to fp32
    assert out.item() == float(np.float32(n))


@pytest.mark.parametrize("op", ["softmax", "rmsnorm"])
def test_rows_past_2g_elements(lib, op):
    rows, cols = 2 ** 21 + 3, 1024
    assert rows * cols > BIG
    x = _randn((rows, cols), 11, scale=3.0 if op == "softmax" else 1.0)
    y = torch.empty_like(x)
    if op == "softmax":
        check(lib.operatorlib_softmax_f32(ptr(x), ptr(y), rows, cols, stream_handle()), op)
    else:
        w = torch.rand(cols, device="cuda") + 0.5
        check(lib.operatorlib_rmsnorm_f32(ptr(x), ptr(w), ptr(y), rows, cols, 1e-6,
                                          stream_handle()), op)
    torch.cuda.synchronize()
    r = torch.from_numpy(_rows(rows, 12)).cuda()
    xs = x[r].cpu().numpy()
    ys = y[r].cpu().numpy().astype(np.float64)
    ref = oracle.softmax(xs) if op == "softmax" else oracle.rmsnorm(xs, w.cpu().numpy(), 1e-6)
    rel = np.abs(ys - ref) / np.maximum(np.abs(ref), 1e-30)
    assert rel.max() <= 1e-5


@pytest.mark.parametrize("op", ["softmax", "rmsnorm"])
def test_long_rows_past_the_grid_y_limit(lib, op):
    # Rows past 32768 columns are split over workgroups, one grid row per
    # matrix row: more than 65535 of them (the limit of a grid's y and z
    # dimensions) must still launch, and every row be written.
    rows, cols = 65540, 32769
    assert rows * cols > BIG
    x = _randn((rows, cols), 15, scale=3.0 if op == "softmax" else 1.0)
    y = torch.full_like(x, float("nan"))
    if op == "softmax":
        check(lib.operatorlib_softmax_f32(ptr(x), ptr(y), rows, cols, stream_handle()), op)
    else:
        w = torch.rand(cols, device="cuda") + 0.5
        check(lib.operatorlib_rmsnorm_f32(ptr(x), ptr(w), ptr(y), rows, cols, 1e-6,
                                          stream_handle()), op)
    torch.cuda.synchronize()
    assert not torch.isnan(y[-1]).any() and not torch.isnan(y[:, -1]).any()
    r = torch.from_numpy(_rows(rows, 16, 10)).cuda()
    xs = x[r].cpu().numpy()
    ys = y[r].cpu().numpy().astype(np.float64)
    ref = oracle.softmax(xs) if op == "softmax" else oracle.rmsnorm(xs, w.cpu().numpy(), 1e-6)
    rel = np.abs(ys - ref) / np.maximum(np.abs(ref), 1e-30)
    assert rel.max() <= 1e-5
    del x, y


def test_transpose_past_2g_elements(lib):
    n = 46349  # n * n > 2^31; not a multiple of 4: the 4-byte tile kernel
    assert n * n > BIG
    x = _randn((n, n), 13)
    y = torch.empty_like(x)
    check(lib.operatorlib_transpose_f32(ptr(x), ptr(y), n, n, stream_handle()), "transpose")
    torch.cuda.synchronize()
    for r in _rows(n, 14, 12):
        # row r of x is column r of y, bit for bit
        assert torch.equal(y[:, int(r)], x[int(r)]), r


def test_gemm_f16_output_past_2g_elements(lib):
    m = n = 46400
    k = 64
    assert m * n > BIG
    a = _randn((m, k), 15, torch.float16)
    b = _randn((k, n), 16, torch.float16)
    c = torch.empty((m, n), device="cuda")
    check(lib.operatorlib_gemm_f16(ptr(a), ptr(b), ptr(c), m, n, k, stream_handle()),
          "gemm_f16")
    torch.cuda.synchronize()
    rows = _rows(m, 17)
    ref = oracle.gemm(a.float().cpu().numpy(), b.float().cpu().numpy(), rows)
    got = c[torch.from_numpy(rows).cuda()].cpu().numpy()
    assert np.max(np.abs(got - ref)) <= 2e-3


def test_attention_f16_past_2g_elements(lib):
    b, h, s, d = 1, 2049, 8192, 128  # each of Q, K, V holds > 2^31 elements
    assert h * s * d > BIG
    q, k, v = (_randn((b, h, s, d), 20 + i, torch.float16) for i in range(3))
    o = torch.empty((b, h, s, d), device="cuda")
    check(lib.operatorlib_attention_f16(ptr(q), ptr(k), ptr(v), ptr(o), b, h, s, d, 1,
                                        stream_handle()), "attention_f16")
    torch.cuda.synchronize()
    heads = np.array([0, 1, 1024, h - 2, h - 1])
    rows = np.array([0, 1, 4095, s - 2, s - 1])
    hs = torch.from_numpy(heads).cuda()
    sub = [t[0, hs].float().cpu().numpy()[None] for t in (q, k, v)]  # [1, 5, s, d]
    hh = np.repeat(np.arange(len(heads)), len(rows))
    rr = np.tile(rows, len(heads))
    ref = oracle.attention(*sub, True, heads=hh, rows=rr)
    got = o[0, torch.from_numpy(heads[hh]).cuda(), torch.from_numpy(rr).cuda()].cpu().numpy()
    assert np.isfinite(got).all()
    assert np.max(np.abs(got - ref)) <= 2e-3
