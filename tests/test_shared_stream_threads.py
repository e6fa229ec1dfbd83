"""Launchers that use library scratch, driven from two host threads at once.

Every entry point whose launch sequence uses library scratch is called here
through the C ABI (ctypes releases the GIL, so both threads are inside the
library together):
  * reduce_sum_f32 over 1,000,003 values (one fp64 partial per workgroup,
    then the combine kernel);
  * gemm_f16 1 x 4096 x 4096 (decode GEMM, split-K partials + split sum);
  * gemm_f16 1000^3 (K and N not multiples of the fast kernel's steps:
    zero-padded operand copies, then the product);
  * attention_f32 B1 H4 S256 D128 (small grid: keys split over workgroups,
    partials, then the combine kernel).
Each thread has its own inputs and its own output for every call, and
enqueues 50 rounds of the four calls on ONE shared stream: an explicit
stream, the null stream, and hipStreamPerThread (where the two threads'
streams differ although the handle is the same). Every output must match
the oracle to the tolerances of test_gpu_ops.py, and repeated calls must
give identical bits (the launchers are deterministic).

A second test captures the same calls with torch.cuda.graph() on its own
capture stream, after warming them up on a different stream, and replays
the graph while eager calls run on the capture stream.
"""

from __future__ import annotations

import ctypes
import threading

import numpy as np
import pytest
import torch

import oracle
from gpu_util import check, ptr, to_device

pytestmark = pytest.mark.gpu

ROUNDS = 50
HIP_STREAM_PER_THREAD = 2  # hipStreamPerThread, include/hip/hip_runtime_api.h


class Case:
    """One thread's inputs, oracle references and per-round outputs."""

    def __init__(self, seed: int, rounds: int):
        self.x = oracle.uniform(seed, 1_000_003)
        self.a1 = oracle.to_f16_bits(oracle.uniform(seed + 1, (1, 4096)))
        self.b1 = oracle.to_f16_bits(oracle.uniform(seed + 2, (4096, 4096)))
        self.ap = oracle.to_f16_bits(oracle.uniform(seed + 3, (1000, 1000)))
        self.bp = oracle.to_f16_bits(oracle.uniform(seed + 4, (1000, 1000)))
        self.q, self.k, self.v = (oracle.normal(seed + 5 + i, (1, 4, 256, 128)) for i in range(3))
        f = oracle.from_f16_bits
        self.ref = {
            "reduce": oracle.reduce_sum(self.x),
            "skinny": oracle.gemm(f(self.a1), f(self.b1)),
            "padded": oracle.gemm(f(self.ap), f(self.bp)),
            "attn": oracle.attention(self.q, self.k, self.v, False),
        }
        self.dev = {name: to_device(getattr(self, name))
                    for name in ("x", "a1", "b1", "ap", "bp", "q", "k", "v")}
        self.out = {
            "reduce": torch.full((rounds,), float("nan"), device="cuda"),
            "skinny": torch.full((rounds, 1, 4096), float("nan"), device="cuda"),
            "padded": torch.full((rounds, 1000, 1000), float("nan"), device="cuda"),
            "attn": torch.full((rounds, 1, 4, 256, 128), float("nan"), device="cuda"),
        }

    def enqueue(self, lib, stream, r: int) -> None:
        d, o = self.dev, self.out
        check(lib.operatorlib_reduce_sum_f32(ptr(d["x"]), ptr(o["reduce"][r:]), d["x"].numel(),
                                             stream), "reduce")
        check(lib.operatorlib_gemm_f16(ptr(d["a1"]), ptr(d["b1"]), ptr(o["skinny"][r]),
                                       1, 4096, 4096, stream), "gemm_f16 skinny")
        check(lib.operatorlib_gemm_f16(ptr(d["ap"]), ptr(d["bp"]), ptr(o["padded"][r]),
                                       1000, 1000, 1000, stream), "gemm_f16 padded")
        check(lib.operatorlib_attention_f32(ptr(d["q"]), ptr(d["k"]), ptr(d["v"]),
                                            ptr(o["attn"][r]), 1, 4, 256, 128, 0, stream),
              "attention_f32")

    def verify(self, label: str, rounds=None) -> None:
        rounds = range(self.out["reduce"].numel()) if rounds is None else rounds
        red = self.out["reduce"].cpu().numpy()
        sk = self.out["skinny"].cpu().numpy().astype(np.float64)
        pd = self.out["padded"].cpu().numpy().astype(np.float64)
        at = self.out["attn"].cpu().numpy().astype(np.float64)
        ref = self.ref
        for r in rounds:
            where = f"{label} round {r}"
            assert abs(red[r] - ref["reduce"]) <= 1e-5 * abs(ref["reduce"]), where
            assert np.max(np.abs(sk[r] - ref["skinny"])) <= 2e-3, where
            assert np.max(np.abs(pd[r] - ref["padded"])) <= 2e-3, where
            err = np.abs(at[r] - ref["attn"])
            assert np.all(err <= 1e-4 + 1e-4 * np.abs(ref["attn"])), where
            # deterministic: every round gives the first round's bits
            assert red[r] == red[rounds[0]], where
            assert np.array_equal(sk[r], sk[rounds[0]]), where
            assert np.array_equal(pd[r], pd[rounds[0]]), where
            assert np.array_equal(at[r], at[rounds[0]]), where


@pytest.fixture(scope="module")
def cases(device):
    made = [Case(1000, ROUNDS), Case(2000, ROUNDS)]
    torch.cuda.synchronize()
    return made


def _reset(cases) -> None:
    for c in cases:
        for t in c.out.values():
            t.fill_(float("nan"))
    torch.cuda.synchronize()


def _hip_runtime():
    # The HIP runtime torch has loaded (same SONAME, so dlopen returns it).
    rt = ctypes.CDLL("libamdhip64.so.7")
    rt.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    rt.hipStreamSynchronize.restype = ctypes.c_int
    return rt


def _run_two_threads(lib, cases, stream_of) -> None:
    errors = []
    start = threading.Barrier(2)
    rt = _hip_runtime()

    def worker(case):
        try:
            stream = stream_of()
            start.wait(timeout=60)
            for r in range(ROUNDS):
                case.enqueue(lib, stream, r)
            # A thread's hipStreamPerThread stream ends with the thread, so
            # each thread waits for its own work before it exits.
            check(rt.hipStreamSynchronize(stream), "hipStreamSynchronize")
        except Exception as exc:  # reported below
            errors.append(repr(exc))

    threads = [threading.Thread(target=worker, args=(c,)) for c in cases]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=300)
    assert not any(th.is_alive() for th in threads), "worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()


def test_two_threads_one_explicit_stream(lib, cases):
    _reset(cases)
    shared = torch.cuda.Stream()
    handle = ctypes.c_void_p(shared.cuda_stream)
    _run_two_threads(lib, cases, lambda: handle)
    for i, c in enumerate(cases):
        c.verify(f"explicit stream, thread {i}")


def test_two_threads_null_stream(lib, cases):
    _reset(cases)
    _run_two_threads(lib, cases, lambda: ctypes.c_void_p(None))
    for i, c in enumerate(cases):
        c.verify(f"null stream, thread {i}")


def test_two_threads_per_thread_stream(lib, cases):
    _reset(cases)
    _run_two_threads(lib, cases, lambda: ctypes.c_void_p(HIP_STREAM_PER_THREAD))
    for i, c in enumerate(cases):
        c.verify(f"hipStreamPerThread, thread {i}")


def test_capture_without_warmup_on_capture_stream(lib, cases):
    """torch.cuda.graph() captures on its own stream, which never ran these
    launchers eagerly; replays on the current stream overlap eager calls on
    the capture stream that use the stream's own scratch."""
    _reset(cases)
    c0, c1 = cases
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):  # warm-up elsewhere (torch's usual pattern)
        c0.enqueue(lib, ctypes.c_void_p(side.cuda_stream), 0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    ctx = torch.cuda.graph(graph)
    with ctx:
        c0.enqueue(lib, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), 1)
    capture_stream = ctypes.c_void_p(ctx.capture_stream.cuda_stream)
    torch.cuda.synchronize()
    replay_stream = torch.cuda.Stream()
    for rep in range(4):
        c0.out["reduce"][1:2].fill_(float("nan"))
        c0.out["skinny"][1].fill_(float("nan"))
        c0.out["padded"][1].fill_(float("nan"))
        c0.out["attn"][1].fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(replay_stream):
            graph.replay()
        # eager calls with other inputs on the capture stream, concurrently
        for r in range(2 * rep, 2 * rep + 2):
            c1.enqueue(lib, capture_stream, r)
        torch.cuda.synchronize()
        c0.verify(f"graph replay {rep}", rounds=[0, 1])
        c1.verify(f"eager beside replay {rep}", rounds=list(range(2 * rep + 2)))
