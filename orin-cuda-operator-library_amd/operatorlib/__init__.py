"""operatorlib for MI355X — Python entry points.

* ``load_operatorlib()`` registers ``torch.ops.operatorlib.{reduce_sum,
  softmax, transpose, rmsnorm, gemm, attention}`` from the in-tree
  extension. Like the reference's ``python/load_extension.py:17-36``, which
  compiles its CUDA sources on first use, it builds the HIP library and the
  binding with hipcc for gfx950 when they are not built yet
  (``OPERATORLIB_NO_BUILD=1`` turns that off); a build that exists is loaded
  as it is.
* ``clib()`` returns the ``ctypes`` handle of ``liboperatorlib.so`` with the
  C ABI of ``include/operatorlib/operatorlib_c.h`` typed, for callers that
  want the library without the torch layer. It builds on first use in the
  same way.

Both raise if the native library is missing and cannot be built: there is
no fallback implementation.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

from . import _build

LIB_DIR = _build.LIB_DIR
LIBRARY_PATH = _build.LIBRARY
TORCH_EXT_PATH = _build.TORCH_EXT

__all__ = ["build", "load_operatorlib", "clib", "LIBRARY_PATH", "TORCH_EXT_PATH",
           "C_SYMBOLS", "HIP_SUCCESS", "HIP_ERROR_INVALID_VALUE"]

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1

_c = ctypes
# name -> (restype, argtypes); mirrors include/operatorlib/operatorlib_c.h
C_SYMBOLS = {
    "operatorlib_abi_version": (_c.c_int, []),
    "operatorlib_status_string": (_c.c_char_p, [_c.c_int]),
    "operatorlib_reduce_sum_f32": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_size_t, _c.c_void_p]),
    "operatorlib_reduce_sum_f32_noalloc": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_size_t,
                                                      _c.c_void_p]),
    "operatorlib_softmax_f32": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_int, _c.c_int, _c.c_void_p]),
    "operatorlib_softmax_f16": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_int, _c.c_int, _c.c_void_p]),
    "operatorlib_rmsnorm_f16": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int, _c.c_int,
                                           _c.c_float, _c.c_void_p]),
    "operatorlib_transpose_f32": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_int, _c.c_int, _c.c_void_p]),
    "operatorlib_rmsnorm_f32": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int, _c.c_int,
                                           _c.c_float, _c.c_void_p]),
    "operatorlib_gemm_f32": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int, _c.c_int,
                                        _c.c_int, _c.c_void_p]),
    "operatorlib_gemm_f16": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int, _c.c_int,
                                        _c.c_int, _c.c_void_p]),
    "operatorlib_attention_f32": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_void_p,
                                             _c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_int,
                                             _c.c_void_p]),
    "operatorlib_attention_f16": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_void_p,
                                             _c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_int,
                                             _c.c_void_p]),
    # workspace forms: the caller's device memory instead of the GPU's arena
    "operatorlib_reduce_sum_f32_workspace_size": (_c.c_size_t, [_c.c_void_p, _c.c_size_t]),
    "operatorlib_reduce_sum_f32_ws": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_size_t,
                                                 _c.c_void_p, _c.c_size_t, _c.c_void_p]),
    "operatorlib_softmax_f32_workspace_size": (_c.c_size_t, [_c.c_int, _c.c_int]),
    "operatorlib_softmax_f32_ws": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_int, _c.c_int,
                                              _c.c_void_p, _c.c_size_t, _c.c_void_p]),
    "operatorlib_softmax_f16_workspace_size": (_c.c_size_t, [_c.c_int, _c.c_int]),
    "operatorlib_softmax_f16_ws": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_int, _c.c_int,
                                              _c.c_void_p, _c.c_size_t, _c.c_void_p]),
    "operatorlib_rmsnorm_f32_workspace_size": (_c.c_size_t, [_c.c_int, _c.c_int]),
    "operatorlib_rmsnorm_f32_ws": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int,
                                              _c.c_int, _c.c_float, _c.c_void_p, _c.c_size_t,
                                              _c.c_void_p]),
    "operatorlib_rmsnorm_f16_workspace_size": (_c.c_size_t, [_c.c_int, _c.c_int]),
    "operatorlib_rmsnorm_f16_ws": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int,
                                              _c.c_int, _c.c_float, _c.c_void_p, _c.c_size_t,
                                              _c.c_void_p]),
    "operatorlib_gemm_f32_workspace_size": (_c.c_size_t, [_c.c_void_p, _c.c_void_p, _c.c_int,
                                                          _c.c_int, _c.c_int]),
    "operatorlib_gemm_f32_ws": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int,
                                           _c.c_int, _c.c_int, _c.c_void_p, _c.c_size_t,
                                           _c.c_void_p]),
    "operatorlib_gemm_f16_workspace_size": (_c.c_size_t, [_c.c_void_p, _c.c_void_p, _c.c_int,
                                                          _c.c_int, _c.c_int]),
    "operatorlib_gemm_f16_ws": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int,
                                           _c.c_int, _c.c_int, _c.c_void_p, _c.c_size_t,
                                           _c.c_void_p]),
    "operatorlib_attention_f32_workspace_size": (_c.c_size_t, [_c.c_void_p, _c.c_void_p,
                                                               _c.c_void_p, _c.c_void_p,
                                                               _c.c_int, _c.c_int, _c.c_int,
                                                               _c.c_int, _c.c_int]),
    "operatorlib_attention_f32_ws": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p,
                                                _c.c_void_p, _c.c_int, _c.c_int, _c.c_int,
                                                _c.c_int, _c.c_int, _c.c_void_p, _c.c_size_t,
                                                _c.c_void_p]),
    "operatorlib_attention_f16_workspace_size": (_c.c_size_t, [_c.c_void_p, _c.c_void_p,
                                                               _c.c_void_p, _c.c_void_p,
                                                               _c.c_int, _c.c_int, _c.c_int,
                                                               _c.c_int, _c.c_int]),
    "operatorlib_attention_f16_ws": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p,
                                                _c.c_void_p, _c.c_int, _c.c_int, _c.c_int,
                                                _c.c_int, _c.c_int, _c.c_void_p, _c.c_size_t,
                                                _c.c_void_p]),
}

_clib = None
_torch_loaded = False


def build(verbose: bool = False, torch_binding: bool = True) -> None:
    """Compile every native artefact for gfx950 (see ``_build``)."""
    _build.build(verbose=verbose, torch_binding=torch_binding)


def _require(path: Path, torch_binding: bool) -> None:
    """Build the native artefacts if `path` is missing; raise if that is not
    possible."""
    if path.exists():
        return
    if os.environ.get("OPERATORLIB_NO_BUILD", "0") == "1":
        raise RuntimeError(
            f"operatorlib native library missing: {path} (OPERATORLIB_NO_BUILD=1). "
            "Build it with python -c 'import __graft_entry__ as g; g.build()'.")
    try:
        if torch_binding:
            _build.build(torch_binding=True)
        else:
            _build.build_library()
    except Exception as exc:  # no silent fallback: report and stop
        raise RuntimeError(f"operatorlib native library missing: {path}, and building "
                           f"it failed: {exc}") from exc
    if not path.exists():
        raise RuntimeError(f"operatorlib build did not produce {path}")


def clib() -> ctypes.CDLL:
    """Load ``liboperatorlib.so`` and type its C ABI."""
    global _clib
    if _clib is None:
        _require(LIBRARY_PATH, torch_binding=False)
        try:
            # Share the HIP runtime torch already loaded (same SONAME) when
            # torch is importable, so both use one runtime instance.
            import torch  # noqa: F401
        except ImportError:
            pass
        lib = ctypes.CDLL(str(LIBRARY_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (restype, argtypes) in C_SYMBOLS.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _clib = lib
    return _clib


def load_operatorlib(verbose: bool = False) -> None:
    """Register ``torch.ops.operatorlib.*`` (reference: load_extension.py:17)."""
    global _torch_loaded
    if _torch_loaded:
        return
    import torch
    _require(TORCH_EXT_PATH, torch_binding=True)
    clib()  # the extension links liboperatorlib.so; load it first, same runtime
    torch.ops.load_library(str(TORCH_EXT_PATH))
    if verbose:
        print(f"loaded {TORCH_EXT_PATH}")
    _torch_loaded = True
