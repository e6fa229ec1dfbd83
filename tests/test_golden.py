"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture, and the closed-form fixtures hold
their known answers (iota sum = -500, index-valued transpose, one-hot
softmax rows, constant RMSNorm rows). GPU: the HIP entry points, called
through the C ABI, meet the parity bars against the committed outputs.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def cases(data: dict, suffix: str = "_out") -> list[str]:
    return sorted(k[: -len(suffix)] for k in data if k.endswith(suffix))


def close(a, b, rel=1e-12):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.max(np.abs(a - b), initial=0.0) <= rel * max(np.max(np.abs(b), initial=0.0), 1e-300)


# ----------------------------------------------------------------- CPU side

def test_generator_fixture():
    g = load("generator")
    for seed in (0, 1, 20260809):
        assert np.array_equal(oracle.uniform(seed, 64), g[f"uniform_{seed}"])
        assert np.array_equal(oracle.normal(seed, 64), g[f"normal_{seed}"])


def test_oracle_reproduces_reduce_fixture():
    g = load("reduce")
    assert float(g["iota_out"]) == -500.0          # tests/core_ops_smoke.cu:33-36
    for c in cases(g):
        assert oracle.reduce_sum(g[f"{c}_in"]) == float(g[f"{c}_out"])


def test_oracle_reproduces_softmax_fixture():
    g = load("softmax")
    onehot = g["onehot_out"]
    assert np.array_equal(onehot, (g["onehot_in"] > 0).astype(np.float64))
    for c in cases(g):
        assert close(oracle.softmax(g[f"{c}_in"]), g[f"{c}_out"])


def test_oracle_reproduces_transpose_fixture():
    g = load("transpose")
    r, c = np.meshgrid(np.arange(37), np.arange(65), indexing="ij")
    assert np.array_equal(g["index37x65_out"], (r * 65 + c).T.astype(np.float32))
    for k in cases(g):
        assert np.array_equal(oracle.transpose(g[f"{k}_in"]), g[f"{k}_out"])


def test_oracle_reproduces_rmsnorm_fixture():
    g = load("rmsnorm")
    eps = float(np.float32(1e-5))                    # epsilon crosses the ABI as fp32
    for row, c0 in ((0, 0.5), (1, -2.0)):            # c / sqrt(c^2 + eps)
        want = c0 / np.sqrt(c0 * c0 + eps)
        assert np.allclose(g["const_out"][row], want, rtol=4e-16, atol=0)
    for c in cases(g):
        got = oracle.rmsnorm(g[f"{c}_in"], g[f"{c}_w"], float(g[f"{c}_eps"]))
        assert close(got, g[f"{c}_out"])


def test_oracle_reproduces_gemm_fixture():
    g = load("gemm")
    for c in cases(g):
        a, b = g[f"{c}_a"], g[f"{c}_b"]
        if c.startswith("f16"):
            a, b = oracle.from_f16_bits(a), oracle.from_f16_bits(b)
        assert close(oracle.gemm(a, b), g[f"{c}_out"])


def test_oracle_reproduces_attention_fixture():
    g = load("attention")
    for c in cases(g):
        q, k, v = (g[f"{c}_{t}"] for t in "qkv")
        if c.startswith("f16"):
            q, k, v = (oracle.from_f16_bits(t) for t in (q, k, v))
        causal = "_c1_" in c
        assert close(oracle.attention(q, k, v, causal), g[f"{c}_out"])


# ----------------------------------------------------------------- GPU side

@pytest.fixture(scope="module")
def hip(lib):
    from gpu_util import HipOps
    return HipOps(lib)


@pytest.mark.gpu
def test_hip_reduce_golden(hip):
    g = load("reduce")
    for c in cases(g):
        ref = float(g[f"{c}_out"])
        assert abs(hip.reduce_sum(g[f"{c}_in"]) - ref) <= 1e-5 * abs(ref), c


@pytest.mark.gpu
def test_hip_softmax_golden(hip):
    g = load("softmax")
    for c in cases(g):
        y, ref = hip.softmax(g[f"{c}_in"]), g[f"{c}_out"]
        assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref)), c
        assert np.linalg.norm(y - ref) <= 1e-5 * np.linalg.norm(ref), c


@pytest.mark.gpu
def test_hip_transpose_golden(hip):
    g = load("transpose")
    for c in cases(g):
        assert np.array_equal(hip.transpose(g[f"{c}_in"]), g[f"{c}_out"]), c


@pytest.mark.gpu
def test_hip_rmsnorm_golden(hip):
    g = load("rmsnorm")
    for c in cases(g):
        y = hip.rmsnorm(g[f"{c}_in"], g[f"{c}_w"], float(g[f"{c}_eps"]))
        ref = g[f"{c}_out"]
        assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref)), c
        assert np.linalg.norm(y - ref) <= 1e-5 * np.linalg.norm(ref), c


@pytest.mark.gpu
def test_hip_gemm_golden(hip):
    g = load("gemm")
    for c in cases(g):
        ref = g[f"{c}_out"]
        if c.startswith("f16"):
            y = hip.gemm_f16(g[f"{c}_a"], g[f"{c}_b"])
            assert np.max(np.abs(y - ref)) <= 2e-3, c
        else:
            y = hip.gemm_f32(g[f"{c}_a"], g[f"{c}_b"])
            assert np.linalg.norm(y - ref) <= 1e-4 * np.linalg.norm(ref), c


@pytest.mark.gpu
def test_hip_attention_golden(hip):
    g = load("attention")
    for c in cases(g):
        q, k, v = (g[f"{c}_{t}"] for t in "qkv")
        causal = "_c1_" in c
        ref = g[f"{c}_out"]
        y = hip.attention(q, k, v, causal)
        if c.startswith("f16"):
            # P is rounded to fp16 before P.V; the +-20 "extreme" inputs use
            # the reference's 2e-2 (tests/attention_smoke.cu:154)
            assert np.max(np.abs(y - ref)) <= (2e-2 if c.endswith("_x1") else 2e-3), c
        else:
            assert np.all(np.abs(y - ref) <= 1e-4 + 1e-4 * np.abs(ref)), c
