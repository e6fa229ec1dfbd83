"""Host C++ layers under AddressSanitizer and UndefinedBehaviorSanitizer (CPU).

The reference ran NVIDIA's compute-sanitizer by hand and keeps no script for
it. Here the host-side code is built with ASan + UBSan on every CPU test run:

* the argument predicates every C-ABI entry point evaluates before any HIP
  call (csrc/validate.hpp), at boundary values: tests/host/validate_check.cpp;
* the standalone runner (runner/operatorlib_run.cpp), built by hipcc with the
  sanitizers on its host pass only (-Xarch_host), through the paths that
  end before the first HIP call: usage, a stray argument, an unknown op.

Device code is not sanitized: GPU ASan needs xnack+ code objects, which the
MI355X boxes used here do not run.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

import operatorlib

REPO = Path(__file__).resolve().parents[1]
CSRC = REPO / "orin-cuda-operator-library_amd" / "csrc"
RUNNER_SRC = REPO / "orin-cuda-operator-library_amd" / "runner" / "operatorlib_run.cpp"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SAN_ENV = {**os.environ, "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0",
           "UBSAN_OPTIONS": "print_stacktrace=1"}
SAN_MARKERS = ("AddressSanitizer", "runtime error:", "UndefinedBehaviorSanitizer")


def _no_sanitizer_report(proc: subprocess.CompletedProcess) -> None:
    text = proc.stdout + proc.stderr
    assert not any(m in text for m in SAN_MARKERS), text


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_predicates_under_asan_ubsan(tmp_path):
    exe = tmp_path / "validate_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=all", f"-I{CSRC}",
                    str(REPO / "tests" / "host" / "validate_check.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True, timeout=300)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60, env=SAN_ENV)
    _no_sanitizer_report(proc)
    assert proc.returncode == 0 and "failures=0" in proc.stdout, proc.stdout


@pytest.fixture(scope="module")
def sanitized_runner(tmp_path_factory):
    if not Path(HIPCC).exists():
        pytest.skip("needs hipcc")
    lib_dir = operatorlib.LIB_DIR
    if not (lib_dir / "liboperatorlib.so").exists():
        pytest.skip("liboperatorlib.so not built")
    exe = tmp_path_factory.mktemp("runner") / "operatorlib_run_san"
    # Sanitizers on the host pass only: each -fsanitize follows -Xarch_host.
    subprocess.run([HIPCC, "-O1", "-g", "-std=c++17", "--offload-arch=gfx950",
                    "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                    "-Xarch_host", "-fno-sanitize-recover=all",
                    "-I", str(REPO / "include"), str(RUNNER_SRC),
                    f"-L{lib_dir}", "-loperatorlib", f"-Wl,-rpath,{lib_dir}", "-o", str(exe)],
                   check=True, capture_output=True, text=True, timeout=600)
    return exe


@pytest.mark.parametrize("args,message", [
    ([], "usage:"),
    (["softmax", "rows=4"], "unexpected argument: rows=4"),
    (["nonsense", "--n=3"], "unknown op: nonsense"),
    (["gemm_f64", "--m=1", "--n=1", "--k=1"], "unknown op: gemm_f64"),
])
def test_runner_cli_errors_under_asan_ubsan(sanitized_runner, args, message):
    proc = subprocess.run([str(sanitized_runner), *args], capture_output=True, text=True,
                          timeout=120, env=SAN_ENV)
    _no_sanitizer_report(proc)
    assert proc.returncode == 2 and message in proc.stderr, proc.stderr
