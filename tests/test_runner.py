"""The standalone runner (orin-cuda-operator-library_amd/runner): the modes and
key=value output of the reference's tools/run_final_standalone.sh."""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

import operatorlib

REPO = Path(__file__).resolve().parents[1]
SCRIPT = REPO / "orin-cuda-operator-library_amd" / "runner" / "run_standalone.sh"
RUNNER = operatorlib.LIB_DIR / "operatorlib_run"


def test_runner_usage_without_gpu():
    proc = subprocess.run([str(RUNNER)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 2 and "usage:" in proc.stderr


def test_script_rejects_unknown_mode():
    proc = subprocess.run(["bash", str(SCRIPT), "nonsense"], capture_output=True, text=True,
                          timeout=60)
    assert proc.returncode == 2 and "Usage" in proc.stderr


def _run_mode(mode: str, expected_ops: int) -> str:
    print(f"running {SCRIPT} {mode}", flush=True)
    proc = subprocess.run(["bash", str(SCRIPT), mode], capture_output=True, text=True,
                          timeout=600)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    verdicts = [ln for ln in proc.stdout.splitlines() if ln.startswith("correct=")]
    assert len(verdicts) == expected_ops and all(v == "correct=PASS" for v in verdicts)
    return proc.stdout


@pytest.mark.gpu
def test_runner_smoke_mode(device):
    out = _run_mode("smoke", 8)
    assert "op=attention_f16 b=1 h=2 s=37 d=71 causal=1" in out


@pytest.mark.gpu
def test_runner_benchmark_mode(device):
    out = _run_mode("benchmark", 8)
    assert out.startswith("source_commit=")
    assert out.count("effective_bandwidth_GBps=") == 4 and out.count("tflops=") == 4
