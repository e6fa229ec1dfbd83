"""operatorlib_reduce_sum_f32_noalloc against operatorlib_reduce_sum_f32.

The no-allocation entry point runs the same kernels with its partials in a
static device array, so its results must equal the regular entry point's
bit for bit (and therefore meet the reduce bar, rel <= 1e-5 against the
fp64 oracle). Two calls in a row, the second on a smaller input, check that
the array's contents from the first call do not leak into the second.
Argument errors are those of the regular entry point.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from gpu_util import ptr, stream_handle, to_device

pytestmark = pytest.mark.gpu


def _sum(fn, x: torch.Tensor) -> float:
    out = torch.full((1,), float("nan"), device="cuda")
    status = fn(ptr(x), ptr(out), x.numel(), stream_handle())
    assert status == 0, status
    torch.cuda.synchronize()
    return float(out.item())


@pytest.mark.parametrize("offset", [0, 3])
def test_noalloc_matches_regular_entry_point(lib, offset):
    sizes = [16_777_216 + 5, 1_000_003]  # second call smaller (fewer workgroups)
    for i, n in enumerate(sizes):
        x_host = oracle.uniform(900 + i, n)
        x = to_device(x_host, offset)
        ref = oracle.reduce_sum(x_host)
        regular = _sum(lib.operatorlib_reduce_sum_f32, x)
        noalloc = _sum(lib.operatorlib_reduce_sum_f32_noalloc, x)
        assert np.float32(noalloc).tobytes() == np.float32(regular).tobytes(), (n, noalloc, regular)
        assert abs(noalloc - ref) <= 1e-5 * abs(ref), (n, noalloc, ref)


def test_noalloc_small_and_single_workgroup(lib):
    for n in (1, 7, 4097, 2_100_000, 3):
        x_host = oracle.uniform(950 + n, n)
        x = to_device(x_host)
        assert _sum(lib.operatorlib_reduce_sum_f32_noalloc, x) == \
            _sum(lib.operatorlib_reduce_sum_f32, x), n


def test_noalloc_rejects_what_the_regular_entry_point_rejects(lib):
    x = torch.ones(8, device="cuda")
    null = ctypes.c_void_p(None)
    assert lib.operatorlib_reduce_sum_f32_noalloc(null, ptr(x), 8, stream_handle()) == 1
    assert lib.operatorlib_reduce_sum_f32_noalloc(ptr(x), null, 8, stream_handle()) == 1
    assert lib.operatorlib_reduce_sum_f32_noalloc(ptr(x), ptr(x), 0, stream_handle()) == 1
