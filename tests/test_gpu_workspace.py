"""The *_ws entry points (GPU): a caller workspace instead of the arena.

Every plan that fits the arena is the plan an unlimited workspace gives, so
a *_ws call with exactly the queried bytes must return the plain entry
point's bits; a workspace one byte short must be rejected before anything
is enqueued (the output keeps its NaN fill). Cases: every launch sequence
that uses scratch (reduce partials, decode split-K partials on both skinny
kernels, padded fp16 operands at the 4095^3 BASELINE edge shape, the split
last round of 256 x 256-tile fp16 and fp32 grids, small grids split along
K, split fp32 and fp16 register-staged attention, softmax and RMSNorm rows
split over workgroups).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from gpu_util import empty, ptr, stream_handle, to_device

pytestmark = pytest.mark.gpu

INVALID = 1


def _ws(nbytes: int) -> torch.Tensor:
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")


def _both(plain, ws_call, query, out) -> torch.Tensor:
    """Runs the plain call, then the *_ws call with exactly `query` bytes,
    then with one byte less; compares bits and the rejection. Returns the
    plain call's output."""
    assert plain(stream_handle()) == 0
    torch.cuda.synchronize()
    first = out.clone()
    need = query()
    out.fill_(float("nan"))
    ws = _ws(need)
    assert ws_call(ptr(ws), need, stream_handle()) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, first)
    if need > 0:
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        assert ws_call(ptr(ws), need - 1, stream_handle()) == INVALID
        torch.cuda.synchronize()
        assert torch.isnan(out).all()
    return first


@pytest.mark.parametrize("n", [1_000_003, 1 << 24])
def test_reduce_ws_matches_plain(lib, n):
    x = to_device(oracle.uniform(70, n))
    out = empty((1,))
    y = _both(lambda s: lib.operatorlib_reduce_sum_f32(ptr(x), ptr(out), n, s),
              lambda w, b, s: lib.operatorlib_reduce_sum_f32_ws(ptr(x), ptr(out), n, w, b, s),
              lambda: lib.operatorlib_reduce_sum_f32_workspace_size(ptr(x), n), out)
    ref = oracle.reduce_sum(x.cpu().numpy())
    assert abs(y.item() - ref) <= 1e-5 * abs(ref)


# (rows, cols): few long rows split over workgroups, rows past 32768
# columns (one segment each), and shapes that need no scratch.
ROW_CASES = [(1, 1 << 20), (32, 50257), (63, 5000), (600, 40003), (4096, 1024), (100000, 8)]


@pytest.mark.parametrize("rows,cols", ROW_CASES)
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_softmax_ws_matches_plain(lib, rows, cols, dtype):
    x = oracle.normal(80, (rows, cols), 0.0, 3.0)
    if dtype == "f16":
        d = to_device(oracle.to_f16_bits(x))
        out = torch.full((rows, cols), float("nan"), dtype=torch.float16, device="cuda")
    else:
        d, out = to_device(x), empty((rows, cols))
    plain = getattr(lib, f"operatorlib_softmax_{dtype}")
    ws = getattr(lib, f"operatorlib_softmax_{dtype}_ws")
    query = getattr(lib, f"operatorlib_softmax_{dtype}_workspace_size")
    _both(lambda s: plain(ptr(d), ptr(out), rows, cols, s),
          lambda w, b, s: ws(ptr(d), ptr(out), rows, cols, w, b, s),
          lambda: query(rows, cols), out)


@pytest.mark.parametrize("rows,cols", ROW_CASES)
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_rmsnorm_ws_matches_plain(lib, rows, cols, dtype):
    x = oracle.normal(81, (rows, cols))
    w = oracle.uniform(82, cols, 0.5, 1.5)
    if dtype == "f16":
        d, dw = to_device(oracle.to_f16_bits(x)), to_device(oracle.to_f16_bits(w))
        out = torch.full((rows, cols), float("nan"), dtype=torch.float16, device="cuda")
    else:
        d, dw, out = to_device(x), to_device(w), empty((rows, cols))
    plain = getattr(lib, f"operatorlib_rmsnorm_{dtype}")
    ws = getattr(lib, f"operatorlib_rmsnorm_{dtype}_ws")
    query = getattr(lib, f"operatorlib_rmsnorm_{dtype}_workspace_size")
    _both(lambda s: plain(ptr(d), ptr(dw), ptr(out), rows, cols, 1e-6, s),
          lambda wp, b, s: ws(ptr(d), ptr(dw), ptr(out), rows, cols, 1e-6, wp, b, s),
          lambda: query(rows, cols), out)


# (m, n, k, dtype): narrow decode shapes (split K) on both skinny kernels,
# padded fp16 operands (4095^3), unaligned operands read in place (1000^3,
# 999 x 1001 x 1003, 4095^3 fp32, 500 x 500 x 999), 272-tile fp16 and fp32
# grids whose last round is split, an unaligned grid with a split last round
# (4097 x 4095 x 4093), small grids split along K (64 x 4096 x 4096,
# 1000^3), shapes that need no scratch.
GEMM_CASES = [(1, 1024, 4096, "f16"), (16, 1024, 4096, "f16"), (1, 1024, 4096, "f32"),
              (16, 1024, 4096, "f32"), (1000, 1000, 1000, "f16"), (4095, 4095, 4095, "f16"),
              (4352, 4096, 512, "f16"), (4352, 4096, 512, "f32"), (1024, 1024, 1024, "f16"),
              (999, 1001, 1003, "f32"), (4095, 4095, 4095, "f32"), (4097, 4095, 4093, "f32"),
              (500, 500, 999, "f32"), (64, 4096, 4096, "f16"), (64, 4096, 4096, "f32")]


@pytest.mark.parametrize("m,n,k,dtype", GEMM_CASES)
def test_gemm_ws_matches_plain(lib, m, n, k, dtype):
    a = oracle.uniform(71 + m, (m, k))
    b = oracle.uniform(72 + n, (k, n))
    if dtype == "f16":
        a, b = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
    da, db = to_device(a), to_device(b)
    out = empty((m, n))
    plain = getattr(lib, f"operatorlib_gemm_{dtype}")
    wsf = getattr(lib, f"operatorlib_gemm_{dtype}_ws")
    query = getattr(lib, f"operatorlib_gemm_{dtype}_workspace_size")
    y = _both(lambda s: plain(ptr(da), ptr(db), ptr(out), m, n, k, s),
              lambda w, nb, s: wsf(ptr(da), ptr(db), ptr(out), m, n, k, w, nb, s),
              lambda: query(ptr(da), ptr(db), m, n, k), out)
    rows = np.array(sorted({0, m - 1, m // 2} | set(range(0, m, 256))), dtype=np.int32)
    af = oracle.from_f16_bits(a) if dtype == "f16" else a
    bf = oracle.from_f16_bits(b) if dtype == "f16" else b
    ref = oracle.gemm(af, bf, rows)
    got = y.cpu().numpy().astype(np.float64)[rows]
    if dtype == "f16":
        assert np.max(np.abs(got - ref)) <= 2e-3
    else:
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-4


# head dims that are not whole 16-byte chunks take the register-staged
# kernel, whose small grids split keys through scratch
@pytest.mark.parametrize("dtype,heads,s,d,causal", [("f32", 4, 256, 99, False),
                                                    ("f32", 2, 300, 71, True),
                                                    ("f16", 3, 256, 100, False)])
def test_attention_ws_matches_plain(lib, dtype, heads, s, d, causal):
    q, k, v = (oracle.normal(73 + i, (1, heads, s, d)) for i in range(3))
    if dtype == "f16":
        q, k, v = (oracle.to_f16_bits(t) for t in (q, k, v))
    dq, dk, dv = (to_device(t) for t in (q, k, v))
    out = empty((1, heads, s, d))
    c = int(causal)
    plain = getattr(lib, f"operatorlib_attention_{dtype}")
    wsf = getattr(lib, f"operatorlib_attention_{dtype}_ws")
    query = getattr(lib, f"operatorlib_attention_{dtype}_workspace_size")
    assert query(ptr(dq), ptr(dk), ptr(dv), ptr(out), 1, heads, s, d, c) > 0  # a split grid
    y = _both(lambda st: plain(ptr(dq), ptr(dk), ptr(dv), ptr(out), 1, heads, s, d, c, st),
              lambda w, nb, st: wsf(ptr(dq), ptr(dk), ptr(dv), ptr(out), 1, heads, s, d, c, w,
                                    nb, st),
              lambda: query(ptr(dq), ptr(dk), ptr(dv), ptr(out), 1, heads, s, d, c), out)
    f = oracle.from_f16_bits if dtype == "f16" else (lambda t: t)
    ref = oracle.attention(f(q), f(k), f(v), causal)
    got = y.cpu().numpy().astype(np.float64)
    tol = 2e-3 if dtype == "f16" else 1e-4 + 1e-4 * np.abs(ref)
    assert np.all(np.abs(got - ref) <= tol)
