"""Builds operatorlib's native artefacts in-tree with hipcc for gfx950.

Outputs (all under ``orin-cuda-operator-library_amd/operatorlib/lib``):
  * ``liboperatorlib.so``      — HIP kernels + the C ABI
                                 (include/operatorlib/operatorlib_c.h)
  * ``operatorlib_run``        — standalone key=value runner (runner/)
  * ``_operatorlib_torch.so``  — ``torch.ops.operatorlib.*`` registrations
                                 (same schema as the reference's
                                 python/operatorlib_binding.cpp:190-206)

This replaces the reference's CUDA JIT loader (python/load_extension.py:17-36)
and its CMake build (CMakeLists.txt:16-56): every source is compiled
explicitly for ``--offload-arch=gfx950``; nothing is JIT-compiled at import.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parents[1]          # orin-cuda-operator-library_amd/
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
LIB_DIR = Path(__file__).resolve().parent / "lib"
OBJ_DIR = PKG_ROOT / "_build"

ARCH = os.environ.get("OPERATORLIB_HIP_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Packed-FP32 instructions (v_pk_add/mul/fma_f32) are disabled for device
# code: some of their forms have given silently wrong results on the MI355X
# machines this library is tested on. hipcc's host pass warns that it does not
# know the feature; that warning is filtered below.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
# Line tables (the reference builds with -lineinfo, CMakeLists.txt:30-32) let
# rocprofv3 and other tools map samples to source lines; the gfx950
# instruction stream is the same with and without them.
LINE_TABLES = [] if os.environ.get("OPERATORLIB_LINE_TABLES", "1") == "0" else ["-gline-tables-only"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
                "-I", str(INCLUDE), "-I", str(CSRC)] + DEVICE_FLAGS + LINE_TABLES

LIB_SOURCES = [
    "reduce.hip", "softmax.hip", "rmsnorm.hip", "transpose.hip",
    "gemm.hip", "attention.hip", "scratch.hip", "capi.cpp",
]

LIBRARY = LIB_DIR / "liboperatorlib.so"
TORCH_EXT = LIB_DIR / "_operatorlib_torch.so"


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True)
    noise = "is not a recognized feature for this target"
    out = "\n".join(line for line in proc.stdout.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def _compile(src: Path, obj: Path, extra: list[str], verbose: bool) -> Path:
    obj.parent.mkdir(parents=True, exist_ok=True)
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    _run([HIPCC, *COMMON_FLAGS, *extra, *lang, "-c", str(src), "-o", str(obj)], verbose)
    return obj


def _jobs() -> int:
    return max(1, min(8, int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))


def build_library(verbose: bool = False) -> Path:
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(_jobs()) as pool:
        objs = list(pool.map(
            lambda s: _compile(CSRC / s, OBJ_DIR / (s + ".o"), [], verbose),
            LIB_SOURCES))
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}",
          *[str(o) for o in objs], "-o", str(tmp)], verbose)
    os.replace(tmp, LIBRARY)
    return LIBRARY


def _torch_flags() -> tuple[list[str], list[str]]:
    import torch.utils.cpp_extension as ce  # deferred: only the binding needs torch
    inc = []
    for p in ce.include_paths():
        inc += ["-isystem", p]
    libdir = ce.library_paths()[0]
    abi = int(getattr(__import__("torch")._C, "_GLIBCXX_USE_CXX11_ABI", 1))
    cflags = inc + [f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DUSE_ROCM=1",
                    "-D__HIP_PLATFORM_AMD__=1", "-DTORCH_EXTENSION_NAME=_operatorlib_torch"]
    ldflags = [f"-L{libdir}", f"-Wl,-rpath,{libdir}", "-lc10", "-ltorch", "-ltorch_cpu",
               "-lc10_hip", "-ltorch_hip"]
    return cflags, ldflags


def build_torch_binding(verbose: bool = False) -> Path:
    cflags, ldflags = _torch_flags()
    obj = _compile(CSRC / "torch_binding.cpp", OBJ_DIR / "torch_binding.cpp.o",
                   cflags, verbose)
    tmp = TORCH_EXT.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", str(obj),
          f"-L{LIB_DIR}", "-loperatorlib", "-Wl,-rpath,$ORIGIN", *ldflags,
          "-o", str(tmp)], verbose)
    os.replace(tmp, TORCH_EXT)
    return TORCH_EXT


CALIBRATION = LIB_DIR / "libopl_calibration.so"


def build_calibration(verbose: bool = False) -> Path:
    """HBM streaming kernels bench.py times beside the operators
    (calibration/stream.hip); not part of the operatorlib ABI."""
    src = PKG_ROOT / "calibration" / "stream.hip"
    tmp = CALIBRATION.with_suffix(".so.tmp")
    _run([HIPCC, *COMMON_FLAGS, "-shared", "-x", "hip", str(src), "-o", str(tmp)], verbose)
    os.replace(tmp, CALIBRATION)
    return CALIBRATION


RUNNER = LIB_DIR / "operatorlib_run"


def build_runner(verbose: bool = False) -> Path:
    """The standalone key=value runner (runner/operatorlib_run.cpp)."""
    src = PKG_ROOT / "runner" / "operatorlib_run.cpp"
    tmp = RUNNER.with_name(RUNNER.name + ".tmp")
    _run([HIPCC, *COMMON_FLAGS, str(src), f"-L{LIB_DIR}", "-loperatorlib",
          "-Wl,-rpath,$ORIGIN", "-o", str(tmp)], verbose)
    os.replace(tmp, RUNNER)
    return RUNNER


CMAKE_BUILD_DIR = REPO_ROOT / "build" / "cmake"


def build_cmake(verbose: bool = False, build_dir: Path = CMAKE_BUILD_DIR) -> Path:
    """Configure and build the CMake project (CMakeLists.txt at the repository
    root): liboperatorlib for C++ consumers, the runner, and the smoke
    programs that ``ctest --test-dir <build_dir>`` runs."""
    cmake = shutil.which("cmake")
    if cmake is None:
        raise RuntimeError("cmake not found")
    generator = ["-G", "Ninja"] if shutil.which("ninja") else []
    _run([cmake, "-S", str(REPO_ROOT), "-B", str(build_dir), *generator,
          f"-DCMAKE_HIP_ARCHITECTURES={ARCH}", "-DCMAKE_BUILD_TYPE=Release"], verbose)
    _run([cmake, "--build", str(build_dir), "-j", str(_jobs())], verbose)
    return build_dir


def build(verbose: bool = False, torch_binding: bool = True) -> None:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    build_library(verbose)
    build_runner(verbose)
    build_calibration(verbose)
    if torch_binding:
        build_torch_binding(verbose)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(f"built {LIBRARY}")
