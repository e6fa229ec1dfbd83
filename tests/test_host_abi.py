"""CPU-side checks of the library boundary (no GPU needed, no kernel runs).

* liboperatorlib.so loads and exports every function include/*.h declares;
* the C and C++ headers compile on their own (C99 for the C ABI);
* argument validation rejects the reference's invalid inputs with
  hipErrorInvalidValue before any HIP call (src/reduce.cu:56-57,
  src/softmax.cu:184-185, src/transpose.cu:40-41, src/rmsnorm.cu:80-82,
  src/attention.cu:448-451, :489-492), so it is testable without a device;
* the torch extension registers the reference's schema strings byte for
  byte (python/operatorlib_binding.cpp:190-197);
* the C++ API keeps the reference's function names and order
  (include/operatorlib/operators.h:13-44).
"""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

import operatorlib

REPO = Path(__file__).resolve().parents[1]
INCLUDE = REPO / "include"
C_HEADER = INCLUDE / "operatorlib" / "operatorlib_c.h"
CPP_HEADER = INCLUDE / "operatorlib" / "operators.h"

REFERENCE_SCHEMA = [
    "reduce_sum(Tensor input) -> Tensor",
    "softmax(Tensor input) -> Tensor",
    "transpose(Tensor input) -> Tensor",
    "rmsnorm(Tensor input, Tensor weight, float epsilon=1e-5) -> Tensor",
    "gemm(Tensor a, Tensor b) -> Tensor",
    "attention(Tensor q, Tensor k, Tensor v, bool causal=False) -> Tensor",
]
BINDING_SOURCE = REPO / "orin-cuda-operator-library_amd" / "csrc" / "torch_binding.cpp"

REFERENCE_API = ["reduce_sum_f32", "softmax_f32", "transpose_f32", "rmsnorm_f32",
                 "gemm_f32", "gemm_f16", "attention_f32", "attention_f16"]
# FP16 row-wise launchers: the reference's deferred dtype extension
# (docs/pytorch_extension.md:143-146), not part of its API.
EXTENSION_API = ["softmax_f16", "rmsnorm_f16"]

INVALID = operatorlib.HIP_ERROR_INVALID_VALUE
FAKE = ctypes.c_void_p(0x1000)   # never dereferenced: every call below fails validation
NULL = None


def declared_c_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", C_HEADER.read_text(), flags=re.S)
    return re.findall(r"\b(operatorlib_\w+)\s*\(", text)


@pytest.fixture(scope="module")
def lib():
    return operatorlib.clib()


def test_every_declared_symbol_is_exported(lib):
    names = declared_c_functions()
    assert len(names) == 31, names
    assert set(names) == set(operatorlib.C_SYMBOLS)
    for name in names:
        assert hasattr(lib, name), name


def test_exported_dynamic_symbols_are_exactly_the_abi():
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    out = subprocess.run([nm, "-D", "--defined-only", str(operatorlib.LIBRARY_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines()
                if ln.split() and ln.split()[-1].startswith("operatorlib_")}
    assert exported == set(declared_c_functions())


def test_abi_version_and_status_strings(lib):
    assert lib.operatorlib_abi_version() == 3
    assert lib.operatorlib_status_string(0)
    assert b"invalid" in lib.operatorlib_status_string(INVALID).lower()


def test_c_header_is_plain_c99(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = tmp_path / "abi.c"
    src.write_text("#include <operatorlib/operatorlib_c.h>\n"
                   "int main(void) { return operatorlib_abi_version() == "
                   "OPERATORLIB_ABI_VERSION ? 0 : 1; }\n")
    subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", "-pedantic", "-I", str(INCLUDE),
                    "-c", str(src), "-o", str(tmp_path / "abi.o")], check=True)


def test_cpp_api_names_and_order():
    text = CPP_HEADER.read_text()
    names = re.findall(r"inline\s+hipError_t\s+(\w+)\s*\(", text)
    assert [n for n in names if n in REFERENCE_API] == REFERENCE_API
    assert sorted(names) == sorted(REFERENCE_API + EXTENSION_API)
    assert text.count("hipStream_t stream = nullptr") == len(names)


# -------------------------------------------------- validation before any HIP call

@pytest.mark.parametrize("fn", ["operatorlib_reduce_sum_f32", "operatorlib_reduce_sum_f32_noalloc"])
def test_reduce_rejects(lib, fn):
    f = getattr(lib, fn)
    assert f(NULL, FAKE, 10, NULL) == INVALID
    assert f(FAKE, NULL, 10, NULL) == INVALID
    assert f(FAKE, FAKE, 0, NULL) == INVALID


@pytest.mark.parametrize("fn", ["operatorlib_softmax_f32", "operatorlib_softmax_f16",
                                "operatorlib_transpose_f32"])
@pytest.mark.parametrize("args", [(NULL, FAKE, 4, 4), (FAKE, NULL, 4, 4), (FAKE, FAKE, 0, 4),
                                  (FAKE, FAKE, 4, 0), (FAKE, FAKE, -1, 4), (FAKE, FAKE, 4, -7)])
def test_matrix_ops_reject(lib, fn, args):
    assert getattr(lib, fn)(*args, NULL) == INVALID


@pytest.mark.parametrize("args", [
    (NULL, FAKE, FAKE, 2, 8, 1e-5), (FAKE, NULL, FAKE, 2, 8, 1e-5), (FAKE, FAKE, NULL, 2, 8, 1e-5),
    (FAKE, FAKE, FAKE, 0, 8, 1e-5), (FAKE, FAKE, FAKE, 2, 0, 1e-5),
    (FAKE, FAKE, FAKE, 2, 8, 0.0), (FAKE, FAKE, FAKE, 2, 8, -1e-5),
    (FAKE, FAKE, FAKE, 2, 8, -0.0), (FAKE, FAKE, FAKE, 2, 8, float("-inf"))])
@pytest.mark.parametrize("fn", ["operatorlib_rmsnorm_f32", "operatorlib_rmsnorm_f16"])
def test_rmsnorm_rejects(lib, fn, args):
    assert getattr(lib, fn)(*args, NULL) == INVALID


@pytest.mark.parametrize("fn", ["operatorlib_gemm_f32", "operatorlib_gemm_f16"])
@pytest.mark.parametrize("args", [(NULL, FAKE, FAKE, 4, 4, 4), (FAKE, NULL, FAKE, 4, 4, 4),
                                  (FAKE, FAKE, NULL, 4, 4, 4), (FAKE, FAKE, FAKE, 0, 4, 4),
                                  (FAKE, FAKE, FAKE, 4, 0, 4), (FAKE, FAKE, FAKE, 4, 4, 0)])
def test_gemm_rejects(lib, fn, args):
    assert getattr(lib, fn)(*args, NULL) == INVALID


@pytest.mark.parametrize("fn", ["operatorlib_attention_f32", "operatorlib_attention_f16"])
@pytest.mark.parametrize("args", [
    (NULL, FAKE, FAKE, FAKE, 1, 1, 8, 16), (FAKE, NULL, FAKE, FAKE, 1, 1, 8, 16),
    (FAKE, FAKE, NULL, FAKE, 1, 1, 8, 16), (FAKE, FAKE, FAKE, NULL, 1, 1, 8, 16),
    (FAKE, FAKE, FAKE, FAKE, 0, 1, 8, 16), (FAKE, FAKE, FAKE, FAKE, 1, 0, 8, 16),
    (FAKE, FAKE, FAKE, FAKE, 1, 1, 0, 16), (FAKE, FAKE, FAKE, FAKE, 1, 1, 8, 0),
    (FAKE, FAKE, FAKE, FAKE, 1, 1, 8, 129),
    (FAKE, FAKE, FAKE, FAKE, 65536, 65536, 8, 16)])   # batch * heads > INT32_MAX
def test_attention_rejects(lib, fn, args):
    assert getattr(lib, fn)(*args, 0, NULL) == INVALID


# ------------------------------------------------------------- torch schema

def test_torch_schema_source_is_byte_identical():
    defs = re.findall(r'm\.def\("([^"]*)"\)', BINDING_SOURCE.read_text())
    assert defs == REFERENCE_SCHEMA


def test_torch_schema_matches_reference():
    import torch
    operatorlib.load_operatorlib()
    for text in REFERENCE_SCHEMA:
        name = text.split("(")[0]
        got = getattr(torch.ops.operatorlib, name).default._schema
        assert got == torch._C.parse_schema("operatorlib::" + text), (got, text)


def test_torch_ops_have_no_cpu_kernel():
    """Registered on the CUDA key only, as the reference binding is
    (python/operatorlib_binding.cpp:199-206): no silent CPU path."""
    import torch
    operatorlib.load_operatorlib()
    with pytest.raises(NotImplementedError):
        torch.ops.operatorlib.softmax(torch.ones(2, 2))


def test_bench_refuses_more_than_one_gpu():
    """The bench measures one GPU; any other --gpus value exits with a
    message (status 2) before touching a device."""
    import sys
    proc = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    assert "--gpus 2 is not supported" in proc.stdout + proc.stderr
    assert not proc.stdout.strip().startswith("{")  # no bench line


# ------------------------------------------------------------- workspace forms
# Queries and the *_ws entry points' workspace checks run before any HIP
# call, so they are exercised here with fake (never dereferenced) pointers.
# Shapes on the direct-to-LDS path split a grid's partly filled last round
# by the CU count the runtime reports; without a GPU none is reported and
# nothing is split, so these shapes avoid such rounds or that path.

def test_reduce_workspace_size(lib):
    q = lib.operatorlib_reduce_sum_f32_workspace_size
    assert q(FAKE, 0) == 0
    assert q(FAKE, 100) == 0                      # one workgroup: no partials
    assert q(FAKE, 1_000_003) == 8 * 123          # 250,000 float4 / 2048 per workgroup
    assert q(FAKE, 1 << 24) == 8 * 256            # the grid cap: 2 KiB at most
    assert q(FAKE, (1 << 40)) == 8 * 256


def test_gemm_workspace_size(lib):
    f16 = lib.operatorlib_gemm_f16_workspace_size
    f32 = lib.operatorlib_gemm_f32_workspace_size
    # decode: 32 column blocks of 128 x 16 K splits of 256 rows, fp32 partials
    assert f16(FAKE, FAKE, 1, 4096, 4096) == 16 * 1 * 4096 * 4
    assert f32(FAKE, FAKE, 16, 4096, 4096) == 8 * 16 * 4096 * 4  # 64 blocks of 64 x 8
    # 8 column blocks x 64 K splits of 64 rows
    assert f16(FAKE, FAKE, 1, 1024, 4096) == 64 * 1 * 1024 * 4
    # every other shape reads its operands in place, unaligned ones included,
    # except large fp16 ones whose rows are not 4-byte aligned: those rows
    # are copied into chunk-padded rows first (A [M, K'], B [K, N']; with
    # both copied, K is padded to 64 as well: B [K', N'])
    assert f16(FAKE, FAKE, 4095, 4095, 4095) == 4095 * 4096 * 2  # A only, mid size
    assert f16(FAKE, FAKE, 8191, 8191, 8191) == 8191 * 8192 * 2 + 8192 * 8192 * 2
    assert f16(FAKE, FAKE, 8192, 8192, 8191) == 8192 * 8192 * 2  # A only
    assert f16(FAKE, FAKE, 4096, 4096, 4095) == 0  # A only, below the one-operand size
    assert f16(FAKE, FAKE, 4094, 4094, 4094) == 0  # dword-aligned rows
    assert f32(FAKE, FAKE, 4095, 4095, 4095) == 0
    assert f32(FAKE, FAKE, 4096, 4096, 4096) == 0  # one whole round of 256 tiles
    assert f32(FAKE, FAKE, 500, 500, 999) == 0
    assert f16(FAKE, FAKE, 333, 777, 999) == 0
    assert f32(FAKE, FAKE, 200, 200, 200) == 0
    assert f16(NULL, FAKE, 1, 4096, 4096) == 0  # invalid arguments


def test_rowwise_workspace_size(lib):
    # Rows split over workgroups: 512 target workgroups, segments of at
    # least 2048 elements rounded up to 64; 8 bytes per (row, segment) for
    # softmax, 4 for RMSNorm. Rows of at most 4096 columns, and 64 or more
    # rows of at most 32768, need none; longer rows always split (one
    # segment per row once there are 512 rows).
    for q, pair in ((lib.operatorlib_softmax_f32_workspace_size, 8),
                    (lib.operatorlib_softmax_f16_workspace_size, 8),
                    (lib.operatorlib_rmsnorm_f32_workspace_size, 4),
                    (lib.operatorlib_rmsnorm_f16_workspace_size, 4)):
        assert q(4096, 1024) == 0
        assert q(1 << 20, 8) == 0
        assert q(64, 32768) == 0
        assert q(1, 1 << 20) == pair * 512           # 512 segments of 2048
        assert q(32, 50257) == pair * 32 * 16        # 16 segments of 3200
        assert q(63, 5000) == pair * 63 * 2          # 2 segments of 2560
        assert q(4, 1 << 20) == pair * 4 * 128       # 128 segments of 8192
        assert q(600, 40000) == pair * 600           # one segment per row
        assert q(0, 5000) == 0 and q(3, 0) == 0      # invalid sizes
        assert q(2**31 - 1, 40000) == pair * (2**31 - 1)  # one segment per row


def test_rowwise_ws_reject_short_workspace(lib):
    ws = ctypes.c_void_p(0x100000)
    assert lib.operatorlib_softmax_f32_ws(FAKE, FAKE, 1, 1 << 20, NULL, 0, NULL) == INVALID
    assert lib.operatorlib_softmax_f16_ws(FAKE, FAKE, 32, 50257, ws, 4095, NULL) == INVALID
    assert lib.operatorlib_rmsnorm_f32_ws(FAKE, FAKE, FAKE, 4, 1 << 20, 1e-5, ws, 1024,
                                          NULL) == INVALID
    assert lib.operatorlib_rmsnorm_f16_ws(FAKE, FAKE, FAKE, 63, 5000, 1e-5,
                                          ctypes.c_void_p(0x100000 + 16), 1 << 20,
                                          NULL) == INVALID   # not 256-byte aligned
    # argument checks as in the plain forms
    assert lib.operatorlib_softmax_f32_ws(NULL, FAKE, 4, 4, NULL, 0, NULL) == INVALID
    assert lib.operatorlib_rmsnorm_f32_ws(FAKE, FAKE, FAKE, 4, 4, 0.0, NULL, 0, NULL) == INVALID


@pytest.mark.parametrize("bytes_given", [0, 1000])
def test_gemm_ws_rejects_short_workspace(lib, bytes_given):
    ws = ctypes.c_void_p(0x100000) if bytes_given else NULL
    assert lib.operatorlib_gemm_f32_ws(FAKE, FAKE, FAKE, 16, 4096, 4096, ws, bytes_given,
                                       NULL) == INVALID
    assert lib.operatorlib_gemm_f16_ws(FAKE, FAKE, FAKE, 1, 1024, 4096, ws, bytes_given,
                                       NULL) == INVALID


def test_ws_rejects_misaligned_workspace(lib):
    need = lib.operatorlib_reduce_sum_f32_workspace_size(FAKE, 1 << 24)
    ws = ctypes.c_void_p(0x100000 + 16)  # 16-byte, not 256-byte, aligned
    assert lib.operatorlib_reduce_sum_f32_ws(FAKE, FAKE, 1 << 24, ws, need + 256,
                                             NULL) == INVALID


def test_attention_workspace_size(lib):
    q = lib.operatorlib_attention_f32_workspace_size
    # B1 H4 S256 D99 (not whole 16-byte chunks: register-staged): 8 query
    # blocks of 128 rows; 4 key splits (256 / 8 workgroups capped at 4) of
    # [rows][D + 2]
    assert q(FAKE, FAKE, FAKE, FAKE, 1, 4, 256, 99, 0) == 4 * 4 * 256 * 101 * 4
    # D 128, and any whole number of chunks (D 96: the D 128 instances with
    # zero dims past 96), on aligned tensors: the direct-to-LDS kernel, no
    # scratch
    assert q(FAKE, FAKE, FAKE, FAKE, 1, 4, 256, 128, 0) == 0
    assert q(FAKE, FAKE, FAKE, FAKE, 1, 4, 256, 96, 0) == 0
    assert q(FAKE, FAKE, FAKE, FAKE, 1, 4, 256, 129, 0) == 0  # invalid: D > 128
    h = lib.operatorlib_attention_f16_workspace_size
    assert h(FAKE, FAKE, FAKE, FAKE, 4, 32, 8192, 128, 1) == 0  # fast path: none
