"""Runs the HIP smoke programs (tests/smoke/*.cpp, built by build()).

They are C++ callers of include/operatorlib/operators.h, as the reference's
ctest programs (tests/core_ops_smoke.cu, gemm_smoke.cu, attention_smoke.cu,
CMakeLists.txt:40-56) are callers of its API. Each must exit 0 and report
every check as PASS.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE / "smoke"))
import build as smoke_build  # noqa: E402

PROGRAMS = ["attention_smoke", "core_ops_smoke", "gemm_smoke"]


def test_every_smoke_source_is_listed():
    assert sorted(p.stem for p in (HERE / "smoke").glob("*.cpp")) == PROGRAMS


@pytest.mark.gpu
@pytest.mark.parametrize("name", PROGRAMS)
def test_smoke_program(device, name):
    exe = smoke_build.BIN / name
    assert exe.exists(), f"{exe} not built (run __graft_entry__.build())"
    print(f"running {exe}", flush=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    lines = [ln for ln in proc.stdout.splitlines() if "=" in ln]
    assert lines and all("=PASS" in ln for ln in lines), proc.stdout
    assert lines[-1] == f"{name}=PASS"
