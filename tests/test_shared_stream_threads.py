"""Launchers that use library scratch, driven from two host threads at once.

Every entry point whose launch sequence uses library scratch is called here
through the C ABI (ctypes releases the GIL, so both threads are inside the
library together):
  * reduce_sum_f32 over 1,000,003 values (one fp64 partial per workgroup,
    then the combine kernel);
  * gemm_f16 1 x 1024 x 4096 (decode GEMM, split-K partials + split sum);
  * gemm_f16 1000^3 (64 tiles of 128 x 128, fewer than the CUs: every
    tile split along K into partial tiles, then the split sum);
  * attention_f32 B1 H4 S256 D99 (register-staged on a small grid: keys
    split over workgroups, partials, then the combine kernel);
  * gemm_f16 4352 x 4096 x 512 (272 tiles of 256 x 256: the last round's 16
    tiles are split along K, partial tiles, then the tail sum).
  * softmax_f32 3 x 50001 (rows split over workgroups: per-segment
    partials, then the pass that combines them).
All of them take their scratch from the GPU's arena, which every stream
shares: the arena's event chain must order the two threads' sequences.
Each thread has its own inputs and its own output for every call, and
enqueues 50 rounds of the six calls on ONE shared stream: an explicit
stream, the null stream, and hipStreamPerThread (where the two threads'
streams differ although the handle is the same). Every output must match
the oracle to the tolerances of test_gpu_ops.py, and repeated calls must
give identical bits (the launchers are deterministic).

The capture tests use torch.cuda.graph() on its own capture stream, after
warming up on a different stream:
  * the plain entry points, whose graphs use the arena: replays run in
    stream order with the eager calls, as the C ABI requires;
  * the *_ws entry points with a workspace tensor per graph: replays on one
    stream overlap eager calls on another;
  * twenty graphs of the plain entry points: the library holds no more
    device memory after capturing them than before, and every replay
    matches the eager result bit for bit.
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
SKINNY_N = 1024  # decode GEMM width: 8 column blocks x 64 K splits
HIP_STREAM_PER_THREAD = 2  # hipStreamPerThread, include/hip/hip_runtime_api.h
# Split-tail GEMM: [M, K] x [K, N]; rows checked against the oracle: two in
# every 256-row tile row, its first and last.
TAIL_MK = (4352, 512)
TAIL_N = 4096
# attention head dim: 99 (not a whole number of 16-byte chunks) takes the
# register-staged kernel, whose small grids split keys over workgroups
# through scratch (chunk-multiple dims on aligned tensors take the
# direct-to-LDS kernel, which needs none)
ATTN_D = 99
# softmax rows split over workgroups: per-segment partials in scratch
SPLIT_ROWS = (3, 50001)
TAIL_ROWS = np.array(sorted({r for t in range(0, TAIL_MK[0], 256) for r in (t, t + 255)}),
                     dtype=np.int32)


class Case:
    """One thread's inputs, oracle references and per-round outputs."""

    def __init__(self, seed: int, rounds: int):
        self.x = oracle.uniform(seed, 1_000_003)
        self.a1 = oracle.to_f16_bits(oracle.uniform(seed + 1, (1, 4096)))
        self.b1 = oracle.to_f16_bits(oracle.uniform(seed + 2, (4096, SKINNY_N)))
        self.ap = oracle.to_f16_bits(oracle.uniform(seed + 3, (1000, 1000)))
        self.bp = oracle.to_f16_bits(oracle.uniform(seed + 4, (1000, 1000)))
        self.q, self.k, self.v = (oracle.normal(seed + 5 + i, (1, 4, 256, ATTN_D)) for i in range(3))
        self.at = oracle.to_f16_bits(oracle.uniform(seed + 8, TAIL_MK))
        self.bt = oracle.to_f16_bits(oracle.uniform(seed + 9, (TAIL_MK[1], TAIL_N)))
        self.sm = oracle.normal(seed + 10, SPLIT_ROWS, 0.0, 3.0)
        f = oracle.from_f16_bits
        self.ref = {
            "reduce": oracle.reduce_sum(self.x),
            "skinny": oracle.gemm(f(self.a1), f(self.b1)),
            "split_k": oracle.gemm(f(self.ap), f(self.bp)),
            "attn": oracle.attention(self.q, self.k, self.v, False),
            "tail": oracle.gemm(f(self.at), f(self.bt), TAIL_ROWS),
            "softmax": oracle.softmax(self.sm),
        }
        self.dev = {name: to_device(getattr(self, name))
                    for name in ("x", "a1", "b1", "ap", "bp", "q", "k", "v", "at", "bt", "sm")}
        self.out = {
            "reduce": torch.full((rounds,), float("nan"), device="cuda"),
            "skinny": torch.full((rounds, 1, SKINNY_N), float("nan"), device="cuda"),
            "split_k": torch.full((rounds, 1000, 1000), float("nan"), device="cuda"),
            "attn": torch.full((rounds, 1, 4, 256, ATTN_D), float("nan"), device="cuda"),
            "tail": torch.full((rounds, TAIL_MK[0], TAIL_N), float("nan"), device="cuda"),
            "softmax": torch.full((rounds, *SPLIT_ROWS), float("nan"), device="cuda"),
        }

    def enqueue(self, lib, stream, r: int) -> None:
        d, o = self.dev, self.out
        check(lib.operatorlib_reduce_sum_f32(ptr(d["x"]), ptr(o["reduce"][r:]), d["x"].numel(),
                                             stream), "reduce")
        check(lib.operatorlib_gemm_f16(ptr(d["a1"]), ptr(d["b1"]), ptr(o["skinny"][r]),
                                       1, SKINNY_N, 4096, stream), "gemm_f16 skinny")
        check(lib.operatorlib_gemm_f16(ptr(d["ap"]), ptr(d["bp"]), ptr(o["split_k"][r]),
                                       1000, 1000, 1000, stream), "gemm_f16 split_k")
        check(lib.operatorlib_attention_f32(ptr(d["q"]), ptr(d["k"]), ptr(d["v"]),
                                            ptr(o["attn"][r]), 1, 4, 256, ATTN_D, 0, stream),
              "attention_f32")
        check(lib.operatorlib_gemm_f16(ptr(d["at"]), ptr(d["bt"]), ptr(o["tail"][r]),
                                       TAIL_MK[0], TAIL_N, TAIL_MK[1], stream),
              "gemm_f16 split tail")
        check(lib.operatorlib_softmax_f32(ptr(d["sm"]), ptr(o["softmax"][r]), *SPLIT_ROWS,
                                          stream), "softmax split rows")

    def workspace_bytes(self, lib) -> int:
        """The largest workspace query of the six calls."""
        d = self.dev
        tmp = torch.empty(TAIL_MK[0] * TAIL_N, device="cuda")
        return max(
            lib.operatorlib_reduce_sum_f32_workspace_size(ptr(d["x"]), d["x"].numel()),
            lib.operatorlib_gemm_f16_workspace_size(ptr(d["a1"]), ptr(d["b1"]), 1, SKINNY_N,
                                                    4096),
            lib.operatorlib_gemm_f16_workspace_size(ptr(d["ap"]), ptr(d["bp"]), 1000, 1000,
                                                    1000),
            lib.operatorlib_attention_f32_workspace_size(ptr(d["q"]), ptr(d["k"]), ptr(d["v"]),
                                                         ptr(tmp), 1, 4, 256, ATTN_D, 0),
            lib.operatorlib_gemm_f16_workspace_size(ptr(d["at"]), ptr(d["bt"]), TAIL_MK[0],
                                                    TAIL_N, TAIL_MK[1]),
            lib.operatorlib_softmax_f32_workspace_size(*SPLIT_ROWS))

    def enqueue_ws(self, lib, stream, r: int, ws: torch.Tensor) -> None:
        """The six calls through the *_ws entry points, one after another
        on `stream` in one workspace."""
        d, o = self.dev, self.out
        w, nb = ptr(ws), ws.numel()
        check(lib.operatorlib_reduce_sum_f32_ws(ptr(d["x"]), ptr(o["reduce"][r:]),
                                                d["x"].numel(), w, nb, stream), "reduce_ws")
        check(lib.operatorlib_gemm_f16_ws(ptr(d["a1"]), ptr(d["b1"]), ptr(o["skinny"][r]),
                                          1, SKINNY_N, 4096, w, nb, stream), "gemm_f16_ws skinny")
        check(lib.operatorlib_gemm_f16_ws(ptr(d["ap"]), ptr(d["bp"]), ptr(o["split_k"][r]),
                                          1000, 1000, 1000, w, nb, stream), "gemm_f16_ws split_k")
        check(lib.operatorlib_attention_f32_ws(ptr(d["q"]), ptr(d["k"]), ptr(d["v"]),
                                               ptr(o["attn"][r]), 1, 4, 256, ATTN_D, 0, w, nb,
                                               stream), "attention_f32_ws")
        check(lib.operatorlib_gemm_f16_ws(ptr(d["at"]), ptr(d["bt"]), ptr(o["tail"][r]),
                                          TAIL_MK[0], TAIL_N, TAIL_MK[1], w, nb, stream),
              "gemm_f16_ws split tail")
        check(lib.operatorlib_softmax_f32_ws(ptr(d["sm"]), ptr(o["softmax"][r]), *SPLIT_ROWS,
                                             w, nb, stream), "softmax_ws split rows")

    def verify(self, label: str, rounds=None) -> None:
        rounds = range(self.out["reduce"].numel()) if rounds is None else rounds
        red = self.out["reduce"].cpu().numpy()
        sk = self.out["skinny"].cpu().numpy().astype(np.float64)
        pd = self.out["split_k"].cpu().numpy().astype(np.float64)
        at = self.out["attn"].cpu().numpy().astype(np.float64)
        smx = self.out["softmax"].cpu().numpy().astype(np.float64)
        ref = self.ref
        for r in rounds:
            where = f"{label} round {r}"
            assert abs(red[r] - ref["reduce"]) <= 1e-5 * abs(ref["reduce"]), where
            assert np.max(np.abs(sk[r] - ref["skinny"])) <= 2e-3, where
            assert np.max(np.abs(pd[r] - ref["split_k"])) <= 2e-3, where
            err = np.abs(at[r] - ref["attn"])
            assert np.all(err <= 1e-4 + 1e-4 * np.abs(ref["attn"])), where
            assert np.max(np.abs(smx[r] - ref["softmax"])) <= 1e-6, where
            assert np.array_equal(smx[r], smx[rounds[0]]), where
            # deterministic: every round gives the first round's bits
            assert red[r] == red[rounds[0]], where
            assert np.array_equal(sk[r], sk[rounds[0]]), where
            assert np.array_equal(pd[r], pd[rounds[0]]), where
            assert np.array_equal(at[r], at[rounds[0]]), where
            # the split-tail GEMM: checked on the device (3.5 GiB of rounds)
            tail = self.out["tail"][r]
            got = tail[torch.from_numpy(TAIL_ROWS).long().cuda()].cpu().numpy()
            assert np.max(np.abs(got.astype(np.float64) - ref["tail"])) <= 2e-3, where
            assert torch.equal(tail, self.out["tail"][rounds[0]]), where


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


def _nan_round(case, r: int) -> None:
    for t in case.out.values():
        t[r].fill_(float("nan"))


def _capture(fn):
    """Captures fn(stream handle) with torch.cuda.graph() on torch's own
    capture stream, after a warm-up on another stream (torch's usual
    pattern); returns the graph and the capture stream."""
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        fn(ctypes.c_void_p(side.cuda_stream))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    ctx = torch.cuda.graph(graph)
    with ctx:
        fn(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return graph, ctx.capture_stream


def test_capture_plain_entry_points_replay_in_stream_order(lib, cases):
    """Graphs of the plain entry points use the arena: each replay runs in
    stream order with eager calls that use it too."""
    _reset(cases)
    c0, c1 = cases
    c0.enqueue(lib, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), 0)
    graph, _ = _capture(lambda s: c0.enqueue(lib, s, 1))
    stream = torch.cuda.Stream()
    handle = ctypes.c_void_p(stream.cuda_stream)
    for rep in range(4):
        _nan_round(c0, 1)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
            for r in range(2 * rep, 2 * rep + 2):
                c1.enqueue(lib, handle, r)
            graph.replay()
        torch.cuda.synchronize()
        c0.verify(f"graph replay {rep}", rounds=[0, 1])
        c1.verify(f"eager between replays {rep}", rounds=list(range(2 * rep + 2)))


def test_capture_workspace_entry_points_overlap_eager_calls(lib, cases):
    """Graphs of the *_ws entry points own their scratch (a workspace tensor
    kept alive with the graph): replays on one stream overlap eager calls
    on the capture stream that use the arena."""
    _reset(cases)
    c0, c1 = cases
    ws = torch.empty(c0.workspace_bytes(lib), dtype=torch.uint8, device="cuda")
    c0.enqueue(lib, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), 0)
    graph, capture_stream = _capture(lambda s: c0.enqueue_ws(lib, s, 1, ws))
    eager = ctypes.c_void_p(capture_stream.cuda_stream)
    replay_stream = torch.cuda.Stream()
    for rep in range(4):
        _nan_round(c0, 1)
        torch.cuda.synchronize()
        with torch.cuda.stream(replay_stream):
            graph.replay()
        for r in range(2 * rep, 2 * rep + 2):
            c1.enqueue(lib, eager, r)
        torch.cuda.synchronize()
        c0.verify(f"workspace graph replay {rep}", rounds=[0, 1])
        c1.verify(f"eager beside replay {rep}", rounds=list(range(2 * rep + 2)))


GRAPHS = 20
# Device memory the runtime itself may take for 20 instantiated graphs of
# six calls each (graph objects, kernel arguments); the library adds none.
GRAPH_MEMORY_SLACK = 32 << 20


def test_twenty_graphs_hold_no_library_memory(lib, cases):
    """Capturing the six arena-using calls into 20 graphs leaves library-held
    device memory where it was (the arena is static), and every replay gives
    the eager result's bits."""
    _reset(cases)
    c0 = cases[0]
    current = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    c0.enqueue(lib, current, 0)  # eager result, and the arena's first use
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    reserved0 = torch.cuda.memory_reserved()
    graphs = []
    for g in range(GRAPHS):
        r = 1 + g % (ROUNDS - 1)
        graphs.append((r, _capture(lambda s, r=r: c0.enqueue(lib, s, r))[0]))
    free1, _ = torch.cuda.mem_get_info()
    reserved1 = torch.cuda.memory_reserved()
    held = (free0 - free1) - (reserved1 - reserved0)
    assert held <= GRAPH_MEMORY_SLACK, f"{held} bytes held after {GRAPHS} captures"
    for rep in range(2):
        for r, graph in graphs:
            _nan_round(c0, r)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()  # the program's own sync between replays
            c0.verify(f"graph of round {r}, replay {rep}", rounds=[0, r])
