"""torch.ops.operatorlib on the GPU: the binding's behaviour, case by case.

Follows the reference's extension test (python/test_extension.py:30-168):
the same operators and shapes run on a non-default stream, the same
validation errors must carry the same message substrings, and outputs have
the reference binding's dtypes and shapes (python/operatorlib_binding.cpp:
49, 67, 83, 108, 130-131, 168-169). Results are checked against the CPU
oracle, to the tolerances the kernel tests use (the reference's own
torch-comparison tolerances are looser).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def side_stream(device):
    return torch.cuda.Stream(device=device)


def _dev(a: np.ndarray, dtype=torch.float32) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda", dtype)


def _run(stream, fn):
    """Run fn on `stream` (inputs created there too), wait, return the result."""
    with torch.cuda.stream(stream):
        out = fn()
    stream.synchronize()
    return out


def test_reduce_sum_on_side_stream(ops, side_stream):
    x = oracle.normal(101, 1_000_003)
    out = _run(side_stream, lambda: ops.reduce_sum(_dev(x)))
    assert out.dtype == torch.float32 and out.dim() == 0 and out.is_cuda
    ref = oracle.reduce_sum(x)
    assert abs(out.item() - ref) <= 1e-5 * max(abs(ref), np.abs(x).sum() * 1e-7)


# (3, 50001) and (2, 40000) are split over workgroups: the binding passes a
# workspace from torch's allocator to the *_ws entry point
@pytest.mark.parametrize("rows,cols,scale", [(19, 128, 5.0), (17, 1024, 5.0),
                                             (17, 1003, 1000.0), (3, 50001, 5.0),
                                             (100000, 8, 5.0)])
def test_softmax_on_side_stream(ops, side_stream, rows, cols, scale):
    x = oracle.normal(102 + rows, (rows, cols), 0.0, scale)
    out = _run(side_stream, lambda: ops.softmax(_dev(x)))
    assert out.shape == (rows, cols) and out.dtype == torch.float32
    y = out.cpu().numpy()
    assert np.max(np.abs(y - oracle.softmax(x))) <= 1e-6
    assert np.allclose(y.sum(-1), 1.0, rtol=0, atol=1e-5)


def test_softmax_uses_last_dim_of_nd_input(ops, side_stream):
    x = oracle.normal(103, (3, 5, 257), 0.0, 2.0)
    out = _run(side_stream, lambda: ops.softmax(_dev(x)))
    assert out.shape == x.shape
    assert np.max(np.abs(out.cpu().numpy() - oracle.softmax(x))) <= 1e-6


@pytest.mark.parametrize("rows,cols", [(64, 96), (65, 37)])
def test_transpose_on_side_stream(ops, side_stream, rows, cols):
    x = oracle.normal(104, (rows, cols))
    out = _run(side_stream, lambda: ops.transpose(_dev(x)))
    assert out.shape == (cols, rows)
    assert np.array_equal(out.cpu().numpy(), x.T)


@pytest.mark.parametrize("shape", [(3, 7, 1024), (5, 1003), (2, 40000), (4, 65536)])
def test_rmsnorm_on_side_stream(ops, side_stream, shape):
    x = oracle.normal(105, shape)
    w = oracle.normal(106, shape[-1])
    out = _run(side_stream, lambda: ops.rmsnorm(_dev(x), _dev(w), 1e-5))
    assert out.shape == shape
    ref = oracle.rmsnorm(x, w, 1e-5)
    y = out.cpu().numpy()
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.abs(ref).max()


def test_rmsnorm_default_epsilon(ops, side_stream):
    x = oracle.normal(107, (4, 64), 0.0, 1e-3)   # small rows: eps matters
    w = oracle.uniform(108, 64, 0.5, 1.5)
    out = _run(side_stream, lambda: ops.rmsnorm(_dev(x), _dev(w)))
    ref = oracle.rmsnorm(x, w, 1e-5)
    assert np.max(np.abs(out.cpu().numpy() - ref)) <= 1e-5 * np.abs(ref).max()


GEMM_CASES = [(torch.float32, 128, 64, 32), (torch.float32, 7, 37, 23),
              (torch.float16, 128, 128, 32), (torch.float16, 16, 128, 32),
              (torch.float16, 32, 32, 32), (torch.float16, 17, 19, 23),
              (torch.float16, 256, 256, 128)]


@pytest.mark.parametrize("dtype,m,n,k", GEMM_CASES)
def test_gemm_on_side_stream(ops, side_stream, dtype, m, n, k):
    a = oracle.normal(109 + m, (m, k), 0.0, 0.1)
    b = oracle.normal(110 + n, (k, n), 0.0, 0.1)
    if dtype == torch.float16:
        a, b = oracle.quantize_f16(a), oracle.quantize_f16(b)
    out = _run(side_stream, lambda: ops.gemm(_dev(a, dtype), _dev(b, dtype)))
    assert out.dtype == torch.float32 and out.shape == (m, n)
    y, ref = out.cpu().numpy(), oracle.gemm(a, b)
    if dtype == torch.float16:
        assert np.max(np.abs(y - ref)) <= 2e-3
    else:
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) <= 1e-4


ATTN_CASES = [(torch.float32, 32, 64, False), (torch.float32, 32, 128, True),
              (torch.float32, 37, 71, True), (torch.float16, 32, 64, False),
              (torch.float16, 32, 128, True), (torch.float16, 37, 71, True),
              (torch.float16, 256, 128, True)]


@pytest.mark.parametrize("dtype,s,d,causal", ATTN_CASES)
def test_attention_on_side_stream(ops, side_stream, dtype, s, d, causal):
    shape = (1, 2, s, d)
    q = oracle.normal(111 + s, shape, 0.0, 0.25)
    k = oracle.normal(112 + d, shape, 0.0, 0.25)
    v = oracle.normal(113, shape)
    if dtype == torch.float16:
        q, k, v = (oracle.quantize_f16(t) for t in (q, k, v))
    out = _run(side_stream,
               lambda: ops.attention(_dev(q, dtype), _dev(k, dtype), _dev(v, dtype), causal))
    assert out.dtype == torch.float32 and out.shape == shape
    y, ref = out.cpu().numpy(), oracle.attention(q, k, v, causal)
    if dtype == torch.float16:
        assert np.max(np.abs(y - ref)) <= 2e-3
    else:
        assert np.all(np.abs(y - ref) <= 1e-4 + 1e-4 * np.abs(ref))


def test_attention_default_is_non_causal(ops, side_stream):
    shape = (1, 1, 64, 32)
    q, k, v = (oracle.normal(114 + i, shape) for i in range(3))
    out = _run(side_stream, lambda: ops.attention(_dev(q), _dev(k), _dev(v)))
    ref = oracle.attention(q, k, v, False)
    assert np.all(np.abs(out.cpu().numpy() - ref) <= 1e-4 + 1e-4 * np.abs(ref))


def _raises(fn, text):
    with pytest.raises(RuntimeError) as err:
        fn()
    assert text in str(err.value), str(err.value)


def test_validation_messages(ops, device):
    """The substrings python/test_extension.py:124-168 asserts."""
    cuda = dict(device="cuda")
    _raises(lambda: ops.reduce_sum(torch.ones(8, dtype=torch.float16, **cuda)), "float32")
    _raises(lambda: ops.softmax(torch.randn(8, 16, **cuda)[:, ::2]), "contiguous")
    _raises(lambda: ops.softmax(torch.empty(3, 0, **cuda)), "positive int32")
    _raises(lambda: ops.transpose(torch.randn(2, 3, 4, **cuda)), "2D")
    _raises(lambda: ops.rmsnorm(torch.randn(3, 8, **cuda), torch.randn(7, **cuda), 1e-5),
            "weight length")
    _raises(lambda: ops.gemm(torch.randn(4, 8, **cuda), torch.randn(7, 5, **cuda)),
            "a.size(1)")
    bad = (1, 1, 8, 129)
    _raises(lambda: ops.attention(torch.randn(*bad, **cuda), torch.randn(*bad, **cuda),
                                  torch.randn(*bad, **cuda), False), "at most 128")


def test_validation_extra_cases(ops, device):
    cuda = dict(device="cuda")
    _raises(lambda: ops.softmax(torch.randn(4, 4)), "CUDA")            # host tensor
    _raises(lambda: ops.rmsnorm(torch.randn(3, 8, **cuda), torch.ones(8, **cuda), 0.0),
            "epsilon")
    _raises(lambda: ops.gemm(torch.randn(4, 8, **cuda),
                             torch.randn(8, 5, dtype=torch.float16, **cuda)), "dtype")
    _raises(lambda: ops.gemm(torch.randn(4, 8, dtype=torch.float64, **cuda),
                             torch.randn(8, 5, dtype=torch.float64, **cuda)), "float")
    shape = (1, 2, 8, 16)
    _raises(lambda: ops.attention(torch.randn(*shape, **cuda), torch.randn(1, 2, 9, 16, **cuda),
                                  torch.randn(*shape, **cuda), False), "shape")
