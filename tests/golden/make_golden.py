"""Write the golden fixtures in this folder (inputs + fp64 oracle outputs).

Run from the repository root:  python tests/golden/make_golden.py

The reference holds no fixture files; its tests build inputs from seeds or
closed formulas. Its std::mt19937 + uniform_real_distribution streams are
implementation-defined, so they are not reproduced here. The fixtures use:
  * the reference's portable closed-form inputs: the -500..499 iota of
    tests/core_ops_smoke.cu:33-36 (sum exactly -500), a 37x65 index-valued
    matrix for transpose (tests/core_ops_smoke.cu:94-119), and the
    attention input formula of attention/attention_common.h:82-92;
  * the reference's smoke-test shapes (core_ops_smoke.cu:172-176,
    gemm_smoke.cu:141-148, attention_smoke.cu:165-177);
  * inputs from the oracle's SplitMix64 generator (seed stated per case).
Expected outputs are the oracle's fp64 results. Each .npz holds plain
arrays only (np.load with allow_pickle=False reads it).
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO))

import oracle  # noqa: E402


def attention_formula(b: int, h: int, s: int, d: int, extreme: bool):
    """attention/attention_common.h:82-92: q, k, v from index arithmetic."""
    i = np.arange(b * h * s * d, dtype=np.int64)
    scale = np.float32(20.0 if extreme else 1.0)
    q = scale * (((i * 17 + 3) % 101) - 50).astype(np.float32) / np.float32(100.0)
    k = scale * (((i * 29 + 7) % 103) - 51).astype(np.float32) / np.float32(100.0)
    v = (((i * 43 + 11) % 107) - 53).astype(np.float32) / np.float32(100.0)
    shape = (b, h, s, d)
    return (q.astype(np.float32).reshape(shape), k.astype(np.float32).reshape(shape),
            v.reshape(shape))


def make_generator() -> dict:
    out = {}
    for seed in (0, 1, 20260809):
        out[f"uniform_{seed}"] = oracle.uniform(seed, 64)
        out[f"normal_{seed}"] = oracle.normal(seed, 64)
    return out


def make_reduce() -> dict:
    out = {"iota_in": np.arange(-500, 500, dtype=np.float32)}
    out["iota_out"] = np.array(oracle.reduce_sum(out["iota_in"]))
    for n, seed in ((1, 1), (7, 2), (1000, 3), (4099, 4), (65537, 5)):
        x = oracle.uniform(seed, n)
        out[f"u{n}_in"] = x
        out[f"u{n}_out"] = np.array(oracle.reduce_sum(x))
    return out


def make_softmax() -> dict:
    out = {}
    cases = [("1x1", (1, 1), 6, 1.0), ("3x5", (3, 5), 7, 1.0),
             ("19x128", (19, 128), 8, 5.0), ("17x1024", (17, 1024), 9, 5.0),
             ("17x1003", (17, 1003), 10, 1000.0)]
    for name, shape, seed, scale in cases:
        x = oracle.normal(seed, shape, 0.0, scale)
        out[f"{name}_in"] = x
        out[f"{name}_out"] = oracle.softmax(x)
    onehot = np.full((4, 64), -1000.0, dtype=np.float32)
    onehot[np.arange(4), [0, 17, 40, 63]] = 1000.0
    out["onehot_in"] = onehot
    out["onehot_out"] = oracle.softmax(onehot)
    return out


def make_transpose() -> dict:
    out = {}
    index = np.arange(37 * 65, dtype=np.float32).reshape(37, 65)
    out["index37x65_in"] = index
    out["index37x65_out"] = oracle.transpose(index)
    for name, shape, seed in (("1x7", (1, 7), 11), ("64x65", (64, 65), 12),
                              ("130x3", (130, 3), 13)):
        x = oracle.uniform(seed, shape)
        out[f"{name}_in"] = x
        out[f"{name}_out"] = oracle.transpose(x)
    return out


def make_rmsnorm() -> dict:
    out = {}
    cases = [("17x1003", (17, 1003), 14, 1e-5), ("8x4096", (8, 4096), 15, 1e-5),
             ("3x1", (3, 1), 16, 1e-5), ("5x64_eps1e-6", (5, 64), 17, 1e-6)]
    for name, shape, seed, eps in cases:
        x = oracle.uniform(seed, shape, -3.0, 3.0)
        w = oracle.uniform(seed + 100, shape[-1], 0.5, 1.5)
        out[f"{name}_in"] = x
        out[f"{name}_w"] = w
        out[f"{name}_eps"] = np.array(eps)
        out[f"{name}_out"] = oracle.rmsnorm(x, w, eps)
    const = np.full((2, 16), 0.5, dtype=np.float32)
    const[1] = -2.0
    w = np.ones(16, dtype=np.float32)
    out["const_in"], out["const_w"], out["const_eps"] = const, w, np.array(1e-5)
    out["const_out"] = oracle.rmsnorm(const, w, 1e-5)
    return out


def make_gemm() -> dict:
    out = {}
    f32 = [(1, 256, 64), (16, 128, 64), (128, 64, 32), (37, 65, 71)]
    f16 = [(128, 128, 32), (16, 128, 32), (32, 32, 32), (37, 65, 71)]
    for i, (m, n, k) in enumerate(f32):
        a = oracle.uniform(200 + i, (m, k), -0.25, 0.25)
        b = oracle.uniform(300 + i, (k, n), -0.25, 0.25)
        key = f"f32_{m}x{n}x{k}"
        out[f"{key}_a"], out[f"{key}_b"], out[f"{key}_out"] = a, b, oracle.gemm(a, b)
    for i, (m, n, k) in enumerate(f16):
        a = oracle.to_f16_bits(oracle.uniform(400 + i, (m, k), -0.25, 0.25))
        b = oracle.to_f16_bits(oracle.uniform(500 + i, (k, n), -0.25, 0.25))
        key = f"f16_{m}x{n}x{k}"
        out[f"{key}_a"], out[f"{key}_b"] = a, b
        out[f"{key}_out"] = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b))
    return out


def make_attention() -> dict:
    out = {}
    for s, d, causal, extreme in ((32, 64, False, False), (32, 128, True, False),
                                  (37, 71, True, True)):
        q, k, v = attention_formula(1, 2, s, d, extreme)
        key = f"S{s}_D{d}_c{int(causal)}_x{int(extreme)}"
        out[f"f32_{key}_q"], out[f"f32_{key}_k"], out[f"f32_{key}_v"] = q, k, v
        out[f"f32_{key}_out"] = oracle.attention(q, k, v, causal)
        qh, kh, vh = (oracle.to_f16_bits(t) for t in (q, k, v))
        out[f"f16_{key}_q"], out[f"f16_{key}_k"], out[f"f16_{key}_v"] = qh, kh, vh
        out[f"f16_{key}_out"] = oracle.attention(*(oracle.from_f16_bits(t) for t in (qh, kh, vh)),
                                                 causal)
    return out


MAKERS = {"generator": make_generator, "reduce": make_reduce, "softmax": make_softmax,
          "transpose": make_transpose, "rmsnorm": make_rmsnorm, "gemm": make_gemm,
          "attention": make_attention}


def main() -> None:
    for name, make in MAKERS.items():
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **make())
        print(f"wrote {path.relative_to(REPO)} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
