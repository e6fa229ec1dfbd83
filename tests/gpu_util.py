"""Helpers for GPU tests: run the HIP kernels through the C ABI.

``HipOps`` exposes the same numpy-in / numpy-out calling convention as the
oracle, so tests/pins.py can be applied to the GPU kernels unchanged. Every
call goes through ``liboperatorlib.so``'s ``extern "C"`` entry points on a
torch-allocated device buffer and torch's current HIP stream; an entry point
that returns a non-zero status fails the test.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

_F16 = np.uint16


def ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def stream_handle(stream: torch.cuda.Stream | None = None) -> ctypes.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def to_device(a: np.ndarray, offset: int = 0) -> torch.Tensor:
    """Copy to the GPU; with offset > 0 the returned view starts `offset`
    elements into its allocation (misaligned base pointer)."""
    a = np.ascontiguousarray(a)
    dtype = {np.dtype(np.float32): torch.float32, np.dtype(_F16): torch.float16}[a.dtype]
    flat = torch.empty(a.size + offset, dtype=dtype, device="cuda")
    host = torch.from_numpy(a.view(np.float16) if a.dtype == _F16 else a).reshape(-1)
    flat[offset:].copy_(host.to("cuda"))
    return flat[offset:].view(a.shape)


def empty(shape, offset: int = 0) -> torch.Tensor:
    n = int(np.prod(shape))
    flat = torch.full((n + offset,), float("nan"), dtype=torch.float32, device="cuda")
    return flat[offset:].view(shape)


def check(status: int, name: str) -> None:
    assert status == 0, f"{name} returned status {status}"


class HipOps:
    def __init__(self, lib):
        self.lib = lib

    def reduce_sum(self, x: np.ndarray, offset: int = 0) -> float:
        d = to_device(x.reshape(-1), offset)
        out = empty((1,))
        check(self.lib.operatorlib_reduce_sum_f32(ptr(d), ptr(out), d.numel(),
                                                  stream_handle()), "reduce_sum")
        torch.cuda.synchronize()
        return float(out.item())

    def softmax(self, x: np.ndarray, offset: int = 0) -> np.ndarray:
        rows, cols = x.shape
        d = to_device(x, offset)
        out = empty(x.shape, offset)
        check(self.lib.operatorlib_softmax_f32(ptr(d), ptr(out), rows, cols,
                                               stream_handle()), "softmax")
        torch.cuda.synchronize()
        return out.cpu().numpy().astype(np.float64)

    def transpose(self, x: np.ndarray, offset: int = 0) -> np.ndarray:
        rows, cols = x.shape
        d = to_device(x, offset)
        out = empty((cols, rows), offset)
        check(self.lib.operatorlib_transpose_f32(ptr(d), ptr(out), rows, cols,
                                                 stream_handle()), "transpose")
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def rmsnorm(self, x: np.ndarray, w: np.ndarray, eps: float,
                offset: int = 0) -> np.ndarray:
        hidden = x.shape[-1]
        tokens = x.size // hidden
        d = to_device(x, offset)
        dw = to_device(np.ascontiguousarray(w, np.float32), offset)
        out = empty(x.shape, offset)
        check(self.lib.operatorlib_rmsnorm_f32(ptr(d), ptr(dw), ptr(out), tokens,
                                               hidden, eps, stream_handle()),
              "rmsnorm")
        torch.cuda.synchronize()
        return out.cpu().numpy().astype(np.float64)

    def gemm_f32(self, a: np.ndarray, b: np.ndarray, offset: int = 0) -> np.ndarray:
        m, k = a.shape
        n = b.shape[1]
        da, db = to_device(a, offset), to_device(b, offset)
        out = empty((m, n))
        check(self.lib.operatorlib_gemm_f32(ptr(da), ptr(db), ptr(out), m, n, k,
                                            stream_handle()), "gemm_f32")
        torch.cuda.synchronize()
        return out.cpu().numpy().astype(np.float64)

    def gemm_f16(self, a_bits: np.ndarray, b_bits: np.ndarray,
                 offset: int = 0) -> np.ndarray:
        m, k = a_bits.shape
        n = b_bits.shape[1]
        da, db = to_device(a_bits, offset), to_device(b_bits, offset)
        out = empty((m, n))
        check(self.lib.operatorlib_gemm_f16(ptr(da), ptr(db), ptr(out), m, n, k,
                                            stream_handle()), "gemm_f16")
        torch.cuda.synchronize()
        return out.cpu().numpy().astype(np.float64)

    def attention(self, q, k, v, causal: bool, offset: int = 0) -> np.ndarray:
        """fp32 arrays -> attention_f32; uint16 (fp16 bits) -> attention_f16."""
        b, h, s, d = q.shape
        dq, dk, dv = (to_device(t, offset) for t in (q, k, v))
        out = empty(q.shape, offset)
        fn = (self.lib.operatorlib_attention_f16 if q.dtype == _F16
              else self.lib.operatorlib_attention_f32)
        check(fn(ptr(dq), ptr(dk), ptr(dv), ptr(out), b, h, s, d, int(causal),
                 stream_handle()), "attention")
        torch.cuda.synchronize()
        return out.cpu().numpy().astype(np.float64)
