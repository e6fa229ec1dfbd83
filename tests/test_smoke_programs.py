"""The CMake build (CMakeLists.txt) and the HIP smoke programs ctest runs.

The smoke programs (tests/smoke/*.cpp) are C++ callers of
include/operatorlib/operators.h, as the reference's ctest programs
(tests/core_ops_smoke.cu, gemm_smoke.cu, attention_smoke.cu,
CMakeLists.txt:38-56) are callers of its API.

* CPU: the project configures and builds from scratch with the installed
  cmake into a temporary directory; the CMake-built liboperatorlib.so
  exports every C ABI symbol, and ctest knows the three smoke tests.
* GPU: ctest runs the smoke programs of the in-tree build (build/cmake,
  made by __graft_entry__.build()); each must report every check as PASS.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

import operatorlib
from operatorlib import _build

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
PROGRAMS = ["attention_smoke", "core_ops_smoke", "gemm_smoke"]
C_HEADER = REPO / "include" / "operatorlib" / "operatorlib_c.h"


def test_every_smoke_source_is_registered():
    assert sorted(p.stem for p in (HERE / "smoke").glob("*.cpp")) == PROGRAMS
    text = (REPO / "CMakeLists.txt").read_text()
    assert "foreach(program core_ops_smoke gemm_smoke attention_smoke)" in text


@pytest.fixture(scope="module")
def fresh_cmake_build(tmp_path_factory):
    if shutil.which("cmake") is None:
        pytest.fail("cmake is part of this image and must be found")
    out = tmp_path_factory.mktemp("cmake")
    _build.build_cmake(build_dir=out)
    return out


def test_cmake_build_exports_the_c_abi(fresh_cmake_build):
    lib = fresh_cmake_build / "liboperatorlib.so"
    assert lib.exists()
    exported = subprocess.run(["nm", "-D", "--defined-only", str(lib)],
                              capture_output=True, text=True, check=True).stdout
    names = set(re.findall(r" T (operatorlib_\w+)", exported))
    declared = set(re.findall(r"\b(operatorlib_\w+)\s*\(", C_HEADER.read_text()))
    assert declared and declared <= names, declared - names
    assert declared == set(operatorlib.C_SYMBOLS)


def test_ctest_lists_the_smoke_programs(fresh_cmake_build):
    proc = subprocess.run(["ctest", "--test-dir", str(fresh_cmake_build), "-N"],
                          capture_output=True, text=True, check=True)
    listed = sorted(re.findall(r"Test\s+#\d+: (\S+)", proc.stdout))
    assert listed == sorted(f"operatorlib_{p}" for p in PROGRAMS)


@pytest.mark.gpu
def test_ctest_runs_the_smoke_programs(device):
    build_dir = _build.CMAKE_BUILD_DIR
    assert (build_dir / "CTestTestfile.cmake").exists(), \
        f"{build_dir} not built (run __graft_entry__.build())"
    print(f"ctest --test-dir {build_dir}", flush=True)
    proc = subprocess.run(["ctest", "--test-dir", str(build_dir), "--output-on-failure",
                           "-V"], capture_output=True, text=True, timeout=400)
    print(proc.stdout[-6000:])
    assert proc.returncode == 0, proc.stdout[-6000:] + proc.stderr
    assert "100% tests passed" in proc.stdout
    for name in PROGRAMS:
        assert f"{name}=PASS" in proc.stdout, name
