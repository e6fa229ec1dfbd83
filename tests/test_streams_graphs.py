"""Serving-side behaviour of the launchers (GPU).

* HIP graph capture: every operator, called through torch.ops on the
  capturing stream, is recorded into one graph; the graph is replayed
  several times with eager work and synchronizations between replays, and
  every replay must reproduce the eager results bit for bit (the launchers
  allocate nothing and record no memset nodes; the binding's workspaces
  come from torch's allocator, which under capture serves the graph's own
  pool).
* Concurrency: two host threads launch on two streams at once; both get the
  results a single thread gets (the launchers are reentrant, and the
  binding gives every call a workspace of its own on its stream).
"""

from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _inputs(device):
    g = torch.Generator(device="cpu").manual_seed(7)
    mk = lambda *shape, dtype=torch.float32: torch.randn(*shape, generator=g).to(device, dtype)
    return {
        "x": mk(1_000_003),
        "sm": mk(300, 1003) * 3,
        "tr": mk(520, 260),
        "tr2": mk(1030, 1031),  # 16-byte accesses at 4-byte alignment
        "rn": mk(257, 4096),
        "w": mk(4096).abs() + 0.5,
        "a": mk(300, 640), "b": mk(640, 512),
        "ah": mk(1000, 1000, dtype=torch.float16), "bh": mk(1000, 1000, dtype=torch.float16),
        "a1": mk(1, 4096, dtype=torch.float16), "b1": mk(4096, 4096, dtype=torch.float16),
        "a16": mk(16, 4096, dtype=torch.float16),
        "a12": mk(12, 1024), "b32": mk(1024, 2048),
        "q": mk(1, 4, 256, 128, dtype=torch.float16),
        "k": mk(1, 4, 256, 128, dtype=torch.float16),
        "v": mk(1, 4, 256, 128, dtype=torch.float16),
        # rows split over workgroups (partials in the workspace)
        "sl": mk(3, 50001) * 3, "rl": mk(2, 40000), "wl": mk(40000).abs() + 0.5,
        # head dim 96 on the fast path (dims past 96 zero); head dim 99 on the
        # register-staged kernel
        "q96": mk(1, 4, 256, 96, dtype=torch.float16),
        "k96": mk(1, 4, 256, 96, dtype=torch.float16),
        "v96": mk(1, 4, 256, 96, dtype=torch.float16),
        "q99": mk(1, 4, 256, 99), "k99": mk(1, 4, 256, 99), "v99": mk(1, 4, 256, 99),
    }


def _all_ops(ops, t):
    return [
        ops.reduce_sum(t["x"]),
        ops.softmax(t["sm"]),
        ops.transpose(t["tr"]),
        ops.transpose(t["tr2"]),
        ops.rmsnorm(t["rn"], t["w"], 1e-6),
        ops.softmax(t["sm"].half()),
        ops.rmsnorm(t["rn"].half(), t["w"].half(), 1e-6),
        ops.gemm(t["a"], t["b"]),
        ops.gemm(t["ah"], t["bh"]),      # tiles split along K: workspace partials
        ops.gemm(t["a1"], t["b1"]),      # skinny path with K splits
        ops.gemm(t["a16"], t["b1"]),     # matrix-core skinny kernel, vector A
        ops.gemm(t["a1"], t["b1"][:, :1024].contiguous()),   # narrow: more K splits
        ops.gemm(t["a16"], t["b1"][:, :1024].contiguous()),
        ops.gemm(t["a12"], t["b32"]),    # same, fp32
        ops.attention(t["q"], t["k"], t["v"], True),
        ops.attention(t["q96"], t["k96"], t["v96"], False),
        # fp32 head dim 99 (register-staged), 8 query blocks: keys split over
        # workgroups, partials in the workspace, then the combine kernel
        ops.attention(t["q99"], t["k99"], t["v99"], False),
        ops.softmax(t["sl"]),
        ops.softmax(t["sl"].half()),
        ops.rmsnorm(t["rl"], t["wl"], 1e-6),
    ]


def test_graph_capture_replays_match_eager(ops, device):
    t = _inputs(device)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        eager = [y.clone() for y in _all_ops(ops, t)]
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outs = _all_ops(ops, t)
    for replay in range(4):
        for y in outs:
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (y, e) in enumerate(zip(outs, eager)):
            assert torch.equal(y, e), (replay, i)
        # eager work on the same buffers' neighbours between replays
        _ = ops.softmax(t["sm"] * 0.5)
        torch.cuda.synchronize()


def test_two_threads_two_streams(ops, device):
    t = _inputs(device)
    with torch.cuda.stream(torch.cuda.Stream()):
        single = [y.clone() for y in _all_ops(ops, t)]
    torch.cuda.synchronize()
    results, errors = {}, []

    def worker(name):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                out = None
                for _ in range(5):
                    out = _all_ops(ops, t)
            s.synchronize()
            results[name] = [y.clone() for y in out]
        except Exception as exc:  # reported below
            errors.append(repr(exc))

    threads = [threading.Thread(target=worker, args=(n,)) for n in ("t0", "t1")]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not errors, errors
    for name in ("t0", "t1"):
        for i, (y, e) in enumerate(zip(results[name], single)):
            assert torch.equal(y, e), (name, i)


def test_eager_results_match_oracle_spot_check(ops, device):
    """Anchor the bit-for-bit comparisons above to the oracle."""
    t = _inputs(device)
    y = ops.softmax(t["sm"]).cpu().numpy()
    assert np.max(np.abs(y - oracle.softmax(t["sm"].cpu().numpy()))) <= 1e-6
    r = ops.reduce_sum(t["x"]).item()
    ref = oracle.reduce_sum(t["x"].cpu().numpy())
    assert abs(r - ref) <= 1e-5 * max(abs(ref), 1.0)
    y = ops.softmax(t["sl"]).cpu().numpy()
    assert np.max(np.abs(y - oracle.softmax(t["sl"].cpu().numpy()))) <= 1e-6
    y = ops.rmsnorm(t["rl"], t["wl"], 1e-6).cpu().numpy().astype(np.float64)
    ref = oracle.rmsnorm(t["rl"].cpu().numpy(), t["wl"].cpu().numpy(), 1e-6)
    assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), 1e-30)) <= 1e-5
