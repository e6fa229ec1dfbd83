"""operatorlib CPU oracle — TEST INFRASTRUCTURE ONLY.

numpy/ctypes front end of ``oracle.c``, the plain-C fp64 restatement of the
reference's CPU reference computations (each C function cites the reference
file:line it follows). Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker or the timed CPU baseline — never as an implementation of an
operator. The operatorlib library never loads it.

Pinning (what ties this restatement to the reference's semantics) lives in
``tests/test_oracle.py``: the reference's own known-answer cases (e.g. the
iota reduce of tests/core_ops_smoke.cu:33-36, the iota transpose of
:94-119), closed forms and invariants chosen so that a dropped term, a wrong
sign or index, or a transposed operand fails at least one check, plus
cross-checks against independent numpy/torch float64 computations.
"""

from __future__ import annotations

import ctypes
import subprocess
import threading
from pathlib import Path

import numpy as np

_DIR = Path(__file__).resolve().parent
_LIB_PATH = _DIR / "liboracle.so"
_lock = threading.Lock()
_lib = None

_c = ctypes
_P = _c.c_void_p


def build() -> Path:
    """Compile liboracle.so with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return _LIB_PATH


def use_native_build(directory) -> str:
    """Compile oracle.c with ``-O3 -march=native`` into ``directory`` and
    route every later oracle call through that build; returns the compile
    command. The CPU baseline is quoted for this build.
    ``-ffp-contract=off`` keeps the arithmetic exactly as written, so the
    results are those of the portable build; only the speed differs."""
    global _lib
    out = Path(directory) / "liboracle_native.so"
    cmd = ["gcc", "-O3", "-march=native", "-std=c11", "-fPIC", "-ffp-contract=off",
           "-shared", "-o", str(out), str(_DIR / "oracle.c"), "-lm"]
    subprocess.run(cmd, check=True)
    with _lock:
        _lib = _open(out)
    return " ".join(cmd[:6]) + " oracle.c"


def _load():
    global _lib
    with _lock:
        if _lib is None:
            src_newer = (not _LIB_PATH.exists() or
                         _LIB_PATH.stat().st_mtime < (_DIR / "oracle.c").stat().st_mtime)
            if src_newer:
                build()
            _lib = _open(_LIB_PATH)
    return _lib


def _open(path):
    """Load one build of oracle.c and type its functions."""
    lib = ctypes.CDLL(str(path))
    sig = {
        "oracle_fill_uniform": [_c.c_uint64, _c.c_float, _c.c_float, _P, _c.c_size_t],
        "oracle_fill_normal": [_c.c_uint64, _c.c_float, _c.c_float, _P, _c.c_size_t],
        "oracle_f32_to_f16_array": [_P, _P, _c.c_size_t],
        "oracle_f16_to_f32_array": [_P, _P, _c.c_size_t],
        "oracle_softmax": [_P, _P, _c.c_int, _c.c_int],
        "oracle_transpose": [_P, _P, _c.c_int, _c.c_int],
        "oracle_rmsnorm": [_P, _P, _P, _c.c_int, _c.c_int, _c.c_float],
        "oracle_gemm": [_P, _P, _P, _c.c_int, _c.c_int, _c.c_int, _P, _c.c_int],
        "oracle_attention": [_P, _P, _P, _P, _c.c_int, _c.c_int, _c.c_int, _c.c_int,
                             _P, _P, _c.c_int],
    }
    for name, argtypes in sig.items():
        getattr(lib, name).argtypes = argtypes
        getattr(lib, name).restype = None
    lib.oracle_reduce_sum.argtypes = [_P, _c.c_size_t]
    lib.oracle_reduce_sum.restype = _c.c_double
    return lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_P)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ----------------------------------------------------------------- generator

def uniform(seed: int, shape, lo: float = -1.0, hi: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    _load().oracle_fill_uniform(seed, lo, hi, _ptr(out), out.size)
    return out


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    _load().oracle_fill_normal(seed, mean, std, _ptr(out), out.size)
    return out


def to_f16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    _load().oracle_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out


def from_f16_bits(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    _load().oracle_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


def quantize_f16(x) -> np.ndarray:
    """fp32 -> nearest fp16 (RNE) -> fp32, as the reference does for its FP16
    checks (attention/attention_v6.cu:23-30)."""
    return from_f16_bits(to_f16_bits(x))


# ----------------------------------------------------------------- operators

def reduce_sum(x) -> float:
    x = _f32(x).reshape(-1)
    return float(_load().oracle_reduce_sum(_ptr(x), x.size))


def softmax(x) -> np.ndarray:
    x = _f32(x)
    cols = x.shape[-1]
    rows = x.size // cols
    out = np.empty(x.shape, dtype=np.float64)
    _load().oracle_softmax(_ptr(x), _ptr(out), rows, cols)
    return out


def transpose(x) -> np.ndarray:
    x = _f32(x)
    rows, cols = x.shape
    out = np.empty((cols, rows), dtype=np.float32)
    _load().oracle_transpose(_ptr(x), _ptr(out), rows, cols)
    return out


def rmsnorm(x, w, eps: float) -> np.ndarray:
    x = _f32(x)
    w = _f32(w)
    hidden = x.shape[-1]
    tokens = x.size // hidden
    out = np.empty(x.shape, dtype=np.float64)
    _load().oracle_rmsnorm(_ptr(x), _ptr(w), _ptr(out), tokens, hidden, eps)
    return out


def gemm(a, b, rows=None) -> np.ndarray:
    """fp64 A @ B on fp32 inputs (fp16 callers pass quantized values)."""
    a = _f32(a)
    b = _f32(b)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    if rows is None:
        out = np.empty((m, n), dtype=np.float64)
        _load().oracle_gemm(_ptr(a), _ptr(b), _ptr(out), m, n, k, None, 0)
    else:
        r = np.ascontiguousarray(rows, dtype=np.int32)
        out = np.empty((r.size, n), dtype=np.float64)
        _load().oracle_gemm(_ptr(a), _ptr(b), _ptr(out), m, n, k, _ptr(r), r.size)
    return out


def attention(q, k, v, causal: bool, heads=None, rows=None) -> np.ndarray:
    """fp64 attention on [B, H, S, D] fp32 inputs.

    Without ``heads``/``rows`` returns the full [B, H, S, D] output; with
    them returns [len(rows), D] for the listed (flattened head, row) pairs.
    """
    q, k, v = _f32(q), _f32(k), _f32(v)
    *lead, s, d = q.shape
    bh = int(np.prod(lead)) if lead else 1
    if heads is None:
        out = np.empty((bh * s, d), dtype=np.float64)
        _load().oracle_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(out), bh, s, d,
                                 int(causal), None, None, 0)
        return out.reshape(q.shape)
    h = np.ascontiguousarray(heads, dtype=np.int32)
    r = np.ascontiguousarray(rows, dtype=np.int32)
    assert h.size == r.size
    out = np.empty((r.size, d), dtype=np.float64)
    _load().oracle_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(out), bh, s, d,
                             int(causal), _ptr(h), _ptr(r), r.size)
    return out
