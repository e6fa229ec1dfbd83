"""GPU parity tests: HIP kernels (through the C ABI) against the CPU oracle.

Tolerances (the benchmark contract in BASELINE.json), written here:
  transpose                bit-exact
  reduce                   |y - ref| <= 1e-5 |ref|           (ref fp64)
  softmax, rmsnorm         elementwise max |y-ref|/|ref| over |ref| >= 1e-30,
                           and normwise ||y-ref||/||ref||, each <= 1e-5
  gemm_f32                 ||C - ref||_F / ||ref||_F <= 1e-4
  gemm_f16, attention_f16  max |y - ref| <= 2e-3, ref fp64 on fp16-rounded
                           inputs
  attention_f32            |y - ref| <= 1e-4 + 1e-4 |ref| (the reference's
                           tests/attention_smoke.cu:108 bound)
Small shapes hit every dispatch path of the reference (its smoke-test shape
matrix) and of this library; benchmark shapes run at full size, checked in
full where the oracle is fast and on seeded row samples (always including
the first and last rows) where it is not.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import pins
from gpu_util import HipOps, check, empty, ptr, stream_handle, to_device

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hip(lib):
    return HipOps(lib)


def rel_errors(y: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    mask = np.abs(ref) >= 1e-30
    elem = float(np.max(np.abs(y[mask] - ref[mask]) / np.abs(ref[mask]))) if mask.any() else 0.0
    norm = float(np.linalg.norm((y - ref).ravel()) / max(np.linalg.norm(ref.ravel()), 1e-300))
    return elem, norm


def sample_rows(n: int, count: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    rows = set(rng.choice(n, size=min(count, n), replace=False).tolist())
    rows.update({0, n - 1})
    return np.array(sorted(rows), dtype=np.int32)


# ------------------------------------------------------------------------ reduce

@pytest.mark.parametrize("n", [1, 2, 3, 5, 1000, 1023, 4097, 1_000_003, 16_777_216])
@pytest.mark.parametrize("offset", [0, 1, 3])
def test_reduce_matches_oracle(hip, n, offset):
    x = oracle.uniform(100 + n, n)
    ref = oracle.reduce_sum(x)
    y = hip.reduce_sum(x, offset)
    assert abs(y - ref) <= 1e-5 * abs(ref)
    # design claim: fp64 accumulation -> within one fp32 rounding of ref
    assert abs(y - ref) <= float(np.spacing(np.float32(abs(ref))))


def test_reduce_pins_and_determinism(hip):
    pins.pin_reduce(hip.reduce_sum, tol_rel=1e-7)
    x = oracle.uniform(7, 16_777_216)
    a, b = hip.reduce_sum(x), hip.reduce_sum(x)
    assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)


def test_reduce_two_streams(lib):
    """Reduces on two streams at once share the GPU's arena: its event
    chain orders them on the device, and both sums stay right."""
    from gpu_util import ptr, stream_handle, to_device
    xs = [oracle.uniform(40 + i, 3_000_000) for i in range(2)]
    ds = [to_device(x) for x in xs]
    outs = [torch.empty(1, device="cuda") for _ in xs]
    streams = [torch.cuda.Stream() for _ in xs]
    torch.cuda.synchronize()
    for _ in range(20):
        for d, o, s in zip(ds, outs, streams):
            assert lib.operatorlib_reduce_sum_f32(ptr(d), ptr(o), d.numel(),
                                                  stream_handle(s)) == 0
    torch.cuda.synchronize()
    for x, o in zip(xs, outs):
        ref = oracle.reduce_sum(x)
        assert abs(o.item() - ref) <= 1e-5 * abs(ref)


def test_arena_orders_four_streams(lib):
    """Reduce and split-K decode GEMM calls interleaved over four streams all
    use the GPU's arena; its event chain must order every sequence after the
    previous one, so every output matches the oracle (a missed wait would let
    one call's partials overwrite another's)."""
    from gpu_util import ptr, stream_handle, to_device
    streams = [torch.cuda.Stream() for _ in range(4)]
    xs = [oracle.uniform(90 + i, 1_000_003 + 17 * i) for i in range(4)]
    dx = [to_device(x) for x in xs]
    a = [oracle.to_f16_bits(oracle.uniform(95 + i, (16, 2048))) for i in range(4)]
    b = [oracle.to_f16_bits(oracle.uniform(99 + i, (2048, 1024))) for i in range(4)]
    da, db = [to_device(t) for t in a], [to_device(t) for t in b]
    rounds = 25
    red = torch.full((rounds, 4), float("nan"), device="cuda")
    gem = torch.full((rounds, 4, 16, 1024), float("nan"), device="cuda")
    torch.cuda.synchronize()
    for r in range(rounds):
        for i, st in enumerate(streams):
            h = stream_handle(st)
            assert lib.operatorlib_reduce_sum_f32(ptr(dx[i]), ptr(red[r, i:]), dx[i].numel(),
                                                  h) == 0
            assert lib.operatorlib_gemm_f16(ptr(da[i]), ptr(db[i]), ptr(gem[r, i]), 16, 1024,
                                            2048, h) == 0
    torch.cuda.synchronize()
    red_h = red.cpu().numpy()
    gem_h = gem.cpu().numpy().astype(np.float64)
    for i in range(4):
        ref = oracle.reduce_sum(xs[i])
        gref = oracle.gemm(oracle.from_f16_bits(a[i]), oracle.from_f16_bits(b[i]))
        for r in range(rounds):
            assert abs(red_h[r, i] - ref) <= 1e-5 * abs(ref), (r, i)
            assert red_h[r, i] == red_h[0, i], (r, i)
            assert np.max(np.abs(gem_h[r, i] - gref)) <= 2e-3, (r, i)
            assert np.array_equal(gem_h[r, i], gem_h[0, i]), (r, i)


# ----------------------------------------------------------------------- softmax

SOFTMAX_SHAPES = [(19, 128), (17, 1024), (17, 1003), (5, 1), (3, 7), (1, 4096),
                  (7, 4100), (3, 9000), (2, 32768), (2, 40000), (3, 33333),
                  (4096, 1024), (4097, 1023),
                  # flat 4-row tiles of ragged rows: one short range, a
                  # partial last tile, a single row of the minimum length
                  (4, 9), (6, 1000), (1, 8)]


@pytest.mark.parametrize("shape", SOFTMAX_SHAPES)
@pytest.mark.parametrize("offset", [0, 1, 2, 3])
def test_softmax_matches_oracle(hip, shape, offset):
    x = oracle.normal(200 + shape[1], shape, 0.0, 3.0)
    ref = oracle.softmax(x)
    y = hip.softmax(x, offset)
    elem, norm = rel_errors(y, ref)
    assert elem <= 1e-5 and norm <= 1e-5, (elem, norm)


@pytest.mark.parametrize("shape", [(17, 1003), (19, 128), (4, 5000), (2, 40000)])
def test_softmax_extreme_scale(hip, shape):
    # tests/core_ops_smoke.cu:174: uniform(-1000, 1000) rows; the reference's
    # max-abs 2e-5 and row-sum 2e-5 bounds
    x = oracle.uniform(300, shape, -1000.0, 1000.0)
    ref = oracle.softmax(x)
    y = hip.softmax(x)
    assert np.max(np.abs(y - ref)) <= 2e-5
    assert np.max(np.abs(y.sum(-1) - 1.0)) <= 2e-5


def test_softmax_pins(hip):
    pins.pin_softmax(hip.softmax, tol=2e-7)


# Short rows run G lanes per row (up to 32 elements, or 32 chunks of
# 16-byte aligned rows: vec G = 2, 4 with an idle lane, 32; element G = 1,
# 2, 32); few long rows are split over workgroups, whose (max, sum) pairs
# every workgroup of the row combines in segment order (two-pass rows, and
# register-resident rows when there are fewer than 64).
SOFTMAX_GROUP_SHAPES = [(100000, 8), (4099, 12), (3001, 128), (70001, 1), (65, 2),
                        (20000, 31)]
SOFTMAX_SPLIT_SHAPES = [(1, 1 << 20), (32, 50257), (63, 5000), (5, 131075), (511, 40000)]


@pytest.mark.parametrize("shape", SOFTMAX_GROUP_SHAPES + SOFTMAX_SPLIT_SHAPES)
@pytest.mark.parametrize("offset", [0, 1, 3])
def test_softmax_short_and_split_rows(hip, shape, offset):
    x = oracle.normal(220 + shape[1] % 997, shape, 0.0, 3.0)
    ref = oracle.softmax(x)
    y = hip.softmax(x, offset)
    elem, norm = rel_errors(y, ref)
    assert elem <= 1e-5 and norm <= 1e-5, (elem, norm)


@pytest.mark.parametrize("shape", [(2, 50000), (3, 9000), (700, 8), (700, 5)])
def test_softmax_masked_rows(hip, shape):
    # -inf everywhere but a few columns: whole segments (split rows) and
    # whole lane groups hold only -inf, and must add nothing to the sum.
    rows, cols = shape
    x = np.full(shape, -np.inf, np.float32)
    x[0, cols - 3:] = [0.5, -1.0, 2.0]
    x[1, 1] = 3.0
    x[2:, 0] = oracle.normal(230, rows - 2)
    x[2:, cols - 1] = 1.0
    ref = oracle.softmax(x)
    y = hip.softmax(x)
    assert np.all(np.isfinite(y))
    assert np.max(np.abs(y - ref)) <= 1e-6
    assert np.all(y[x == -np.inf] == 0.0)


# Input and output in different 16-byte phases (rows cannot share one
# float4 layout): the element-wise paths. The weight of RMSNorm may sit at
# any alignment on every path.
MIXED_SHAPES = [(17, 1003), (5, 1), (3, 7), (3, 9000), (4097, 1023), (2, 40000)]


def _rows_call(lib, name, x, in_off, out_off, weight=None, eps=0.0):
    """softmax / rmsnorm through the C ABI with independent input and output
    offsets (elements into their allocations)."""
    from gpu_util import check, empty, ptr, stream_handle, to_device
    d = to_device(x, in_off)
    out = empty(x.shape, out_off)
    rows, cols = x.shape
    fn = getattr(lib, name)
    if weight is None:
        check(fn(ptr(d), ptr(out), rows, cols, stream_handle()), name)
    else:
        check(fn(ptr(d), ptr(weight), ptr(out), rows, cols, eps, stream_handle()), name)
    torch.cuda.synchronize()
    return out.cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("shape", MIXED_SHAPES)
@pytest.mark.parametrize("in_off,out_off", [(1, 0), (0, 3), (2, 1)])
def test_softmax_mixed_phases(lib, shape, in_off, out_off):
    x = oracle.normal(260 + shape[1], shape, 0.0, 3.0)
    y = _rows_call(lib, "operatorlib_softmax_f32", x, in_off, out_off)
    elem, norm = rel_errors(y, oracle.softmax(x))
    assert elem <= 1e-5 and norm <= 1e-5, (elem, norm)


@pytest.mark.parametrize("shape", MIXED_SHAPES)
@pytest.mark.parametrize("in_off,out_off,w_off", [(1, 0, 0), (0, 3, 1), (2, 2, 1), (3, 3, 0)])
def test_rmsnorm_mixed_phases(lib, shape, in_off, out_off, w_off):
    from gpu_util import to_device
    x = oracle.normal(560 + shape[1], shape)
    w = oracle.uniform(561, shape[1], 0.5, 1.5)
    y = _rows_call(lib, "operatorlib_rmsnorm_f32", x, in_off, out_off,
                   to_device(w, w_off), 1e-5)
    elem, norm = rel_errors(y, oracle.rmsnorm(x, w, 1e-5))
    assert elem <= 1e-5 and norm <= 1e-5, (elem, norm)


# --------------------------------------------------------------------- transpose

TRANSPOSE_SHAPES = [(37, 65), (64, 96), (65, 37), (1, 1), (1, 1000), (1000, 1),
                    (64, 64), (129, 257), (4096, 4096), (4095, 4097),
                    # rows, cols % 4 == 0: the float4 kernel, partial 128-tiles
                    (4, 8), (132, 260), (520, 128), (128, 516), (4, 4096), (1024, 4),
                    # tile columns past the last whole strip of 16: 22 (a
                    # partial last tile), 33, 48 (three whole strips)
                    (384, 2700), (1028, 4100), (260, 6144),
                    # >= 64 tiles of 128x128 at any shape (or offset 1): 16-byte
                    # accesses at 4-byte alignment, element-wise edge float4s;
                    # misaligned input rows (cached loads) ...
                    (1030, 1031), (2049, 1027), (1000, 1000),
                    # ... or, at offset 0, aligned input rows and misaligned
                    # output rows (cached stores)
                    (1027, 2048), (4097, 4096),
                    # at most 16 rows or columns: one thread per index of the
                    # long side, 1 to 16 values of the short side each
                    (1, 1 << 20), (1 << 20, 1), (3, 100003), (100003, 3),
                    (8, 4097), (4097, 8), (7, 9), (9, 7), (2, 2),
                    # ... as float4s when the long side is a multiple of 4
                    # (aligned, offset 0): every short side 2..8, both ways
                    (2, 1000), (3, 4096), (5, 1024), (6, 2048), (7, 4100), (8, 65536),
                    (65536, 8), (4100, 7), (2048, 6), (1024, 5), (4096, 3), (1000, 2),
                    (4, 4),
                    # short sides 9..16 (float4 at offset 0 where the long side
                    # is a multiple of 4)
                    (16, 65536), (65536, 16), (12, 4100), (9, 4096), (13, 100003),
                    (4097, 16), (11, 11)]


@pytest.mark.parametrize("shape", TRANSPOSE_SHAPES)
@pytest.mark.parametrize("offset", [0, 1])
def test_transpose_bit_exact(hip, shape, offset):
    x = oracle.uniform(400 + shape[0], shape)
    y = hip.transpose(x, offset)
    ref = oracle.transpose(x)
    assert y.view(np.uint32).tobytes() == ref.view(np.uint32).tobytes()


# Output rows not 16-byte aligned (the line-window kernel), at independent
# input / output phases: offsets in floats past a 16-byte (input) and a
# 128-byte (output) boundary. Rows 1023 and 1022 leave the last 128-row
# block 127 / 126 rows, whose windows run past it; (1024, 1000) has aligned
# row lengths and only a misaligned output base.
WINDOW_SHAPES = [(1000, 1000), (1023, 1025), (1025, 1023), (1022, 1031), (131, 8000),
                 (8000, 131), (1024, 1000), (2047, 2049)]


@pytest.mark.parametrize("shape", WINDOW_SHAPES)
@pytest.mark.parametrize("in_off,out_off", [(0, 5), (3, 17), (2, 31), (1, 0)])
def test_transpose_window_phases(lib, shape, in_off, out_off):
    x = oracle.uniform(430 + shape[1], shape)
    rows, cols = shape
    d = to_device(x, in_off)
    # the output view starts out_off floats past a 256-byte allocation base
    out = empty((cols, rows), out_off)
    check(lib.operatorlib_transpose_f32(ptr(d), ptr(out), rows, cols, stream_handle()),
          "transpose")
    torch.cuda.synchronize()
    y = out.cpu().numpy()
    assert y.view(np.uint32).tobytes() == oracle.transpose(x).view(np.uint32).tobytes()


def test_transpose_pins(hip):
    pins.pin_transpose(hip.transpose)


def test_transpose_involution_full_size(hip):
    x = oracle.uniform(401, (4095, 4097))
    assert np.array_equal(hip.transpose(hip.transpose(x).astype(np.float32)), x)


# ----------------------------------------------------------------------- rmsnorm

RMSNORM_CASES = [((32, 4096), 1e-5), ((17, 1003), 1e-5), ((21, 1024), 1e-5),
                 ((5, 1003), 1e-5), ((3, 1), 1e-5), ((4, 10000), 1e-6),
                 ((2, 32768), 1e-6), ((2, 40001), 1e-6), ((2048, 4096), 1e-6),
                 ((2047, 4095), 1e-6)]


@pytest.mark.parametrize("shape,eps", RMSNORM_CASES)
@pytest.mark.parametrize("offset", [0, 1, 2, 3])
def test_rmsnorm_matches_oracle(hip, shape, eps, offset):
    x = oracle.normal(500 + shape[1], shape)
    w = oracle.uniform(501, shape[1], 0.5, 1.5)
    ref = oracle.rmsnorm(x, w, eps)
    y = hip.rmsnorm(x, w, eps, offset)
    elem, norm = rel_errors(y, ref)
    assert elem <= 1e-5 and norm <= 1e-5, (elem, norm)


def test_rmsnorm_pins(hip):
    pins.pin_rmsnorm(hip.rmsnorm, tol=3e-7)


# Short rows run G lanes per row; few long rows, and every row past 32768
# columns, are split over workgroups whose partial sums of squares the row's
# workgroups add in segment order. The weights sit at the input's offset, so
# odd widths put most rows at another 16-byte phase than the weights.
RMSNORM_GROUP_CASES = [((100000, 16), 1e-6), ((4099, 12), 1e-5), ((3001, 128), 1e-5),
                       ((70001, 1), 1e-5), ((20000, 31), 1e-6)]
RMSNORM_SPLIT_CASES = [((4, 1 << 20), 1e-6), ((64, 65536), 1e-6), ((63, 5000), 1e-5),
                       ((600, 40003), 1e-6)]


@pytest.mark.parametrize("shape,eps", RMSNORM_GROUP_CASES + RMSNORM_SPLIT_CASES)
@pytest.mark.parametrize("offset", [0, 1, 3])
def test_rmsnorm_short_and_split_rows(hip, shape, eps, offset):
    x = oracle.normal(520 + shape[1] % 997, shape)
    w = oracle.uniform(521, shape[1], 0.5, 1.5)
    ref = oracle.rmsnorm(x, w, eps)
    y = hip.rmsnorm(x, w, eps, offset)
    elem, norm = rel_errors(y, ref)
    assert elem <= 1e-5 and norm <= 1e-5, (elem, norm)


def test_rmsnorm_nan_epsilon_is_accepted_as_in_the_reference(lib):
    # The reference launcher rejects only `epsilon <= 0.0f`
    # (src/rmsnorm.cu:80-81), which is false for NaN: the call succeeds and
    # every output is NaN (rsqrt of NaN).
    x = to_device(oracle.normal(61, (3, 40)))
    w = to_device(oracle.uniform(62, 40, 0.5, 1.5))
    out = empty((3, 40))
    check(lib.operatorlib_rmsnorm_f32(ptr(x), ptr(w), ptr(out), 3, 40, float("nan"),
                                      stream_handle()), "rmsnorm")
    torch.cuda.synchronize()
    assert torch.isnan(out).all()


# -------------------------------------------------------------------------- gemm

# The reference smoke matrix (tests/gemm_smoke.cu:141-148) plus shapes that
# exercise this library's fp16 global->LDS path at its M / N edges (K % 32 == 0,
# N % 8 == 0, partial 256-wide tiles) and its fallback paths.
GEMM_SMALL = [(1, 256, 64), (16, 128, 64), (128, 64, 32), (37, 65, 71), (7, 37, 23),
              (128, 128, 32), (16, 128, 32), (32, 32, 32), (17, 19, 23),
              (256, 256, 256), (300, 520, 200), (513, 129, 1000),
              (300, 520, 192), (513, 136, 1024), (1, 8, 64), (1000, 1000, 128)]


@pytest.mark.parametrize("mnk", GEMM_SMALL)
@pytest.mark.parametrize("offset", [0, 1])
def test_gemm_f32_small(hip, mnk, offset):
    m, n, k = mnk
    a = oracle.uniform(600 + m, (m, k))
    b = oracle.uniform(601 + n, (k, n))
    ref = oracle.gemm(a, b)
    y = hip.gemm_f32(a, b, offset)
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) <= 1e-4
    # the reference smoke bound (tests/gemm_smoke.cu:76), elementwise
    assert np.all(np.abs(y - ref) <= 1e-3 + 1e-3 * np.abs(ref))


@pytest.mark.parametrize("mnk", GEMM_SMALL)
@pytest.mark.parametrize("offset", [0, 1])
def test_gemm_f16_small(hip, mnk, offset):
    m, n, k = mnk
    a = oracle.to_f16_bits(oracle.uniform(700 + m, (m, k)))
    b = oracle.to_f16_bits(oracle.uniform(701 + n, (k, n)))
    ref = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b))
    y = hip.gemm_f16(a, b, offset)
    assert np.max(np.abs(y - ref)) <= 2e-3


# M <= 16 (decode shapes): the skinny kernels, with and without K splits,
# partial column blocks and odd K.
GEMM_SKINNY = [(1, 4096, 4096), (4, 4096, 4096), (16, 4096, 4096), (3, 1000, 333),
               (16, 4104, 1000), (1, 8, 5000), (9, 136, 777), (2, 64, 31), (1, 1024, 1),
               # matrix-core variant (M >= 5 fp16, >= 9 fp32): K tails inside
               # a k block, a partial column block, one split
               (5, 264, 1001), (12, 72, 37), (8, 4096, 4096), (13, 520, 4099)]


@pytest.mark.parametrize("mnk", GEMM_SKINNY)
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_gemm_skinny(hip, mnk, dtype):
    m, n, k = mnk
    a = oracle.uniform(640 + m, (m, k))
    b = oracle.uniform(641 + n, (k, n))
    if dtype == "f16":
        ab, bb = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(ab, bb)
        ref = oracle.gemm(oracle.from_f16_bits(ab), oracle.from_f16_bits(bb))
        assert np.max(np.abs(y - ref)) <= 2e-3
    else:
        y = hip.gemm_f32(a, b)
        ref = oracle.gemm(a, b)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) <= 1e-4
        assert np.all(np.abs(y - ref) <= 1e-3 + 1e-3 * np.abs(ref))


@pytest.mark.parametrize("m", [6, 12, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_gemm_skinny_unaligned_a(hip, m, dtype):
    """K % 4 == 0 but A off its 4-element alignment (B aligned, so the
    skinny path still applies): the matrix-core kernel's element-wise A
    loads instead of the vector ones."""
    n, k = 640, 1024
    a = oracle.uniform(660 + m, (m, k))
    b = oracle.uniform(661, (k, n))
    if dtype == "f16":
        a, b = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        fn, ref = hip.lib.operatorlib_gemm_f16, oracle.gemm(oracle.from_f16_bits(a),
                                                             oracle.from_f16_bits(b))
    else:
        fn, ref = hip.lib.operatorlib_gemm_f32, oracle.gemm(a, b)
    da, db = to_device(a, 1), to_device(b)
    out = empty((m, n))
    check(fn(ptr(da), ptr(db), ptr(out), m, n, k, stream_handle()), "gemm")
    torch.cuda.synchronize()
    y = out.cpu().numpy().astype(np.float64)
    if dtype == "f16":
        assert np.max(np.abs(y - ref)) <= 2e-3
    else:
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) <= 1e-4


# M <= 16 at wide N (the LLM decode range): ragged K (a partial last split,
# K below one k block), N off a multiple of the column block, element-wise
# A loads (offset 1), M 1-16; results deterministic.
GEMM_DECODE = [(1, 4104, 1000), (7, 3080, 33), (16, 4096, 4095), (2, 4096, 17),
               (16, 6144, 1024), (1, 3072, 1), (11, 12288, 512), (3, 4112, 4100)]


# Small batches on the matrix-core skinny kernel: two row blocks of 16
# (17..32 rows), four (33..64, fp32; fp16 takes the split 128 x 128 tiles
# there), ragged column blocks (N 4104) and K; misaligned A in
# test_gemm_skinny_unaligned_a.
GEMM_SKINNY_ROWS = [(17, 4104, 1000), (24, 4096, 4096), (32, 136, 777), (33, 4104, 1000),
                    (48, 1000, 333), (64, 4096, 4096)]


@pytest.mark.parametrize("mnk", GEMM_SKINNY_ROWS)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_gemm_skinny_row_blocks(hip, mnk, dtype):
    m, n, k = mnk
    offset = 0
    a = oracle.uniform(670 + m, (m, k))
    b = oracle.uniform(671 + n, (k, n))
    if dtype == "f16":
        a, b = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(a, b, offset)
        ref = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b))
        assert np.max(np.abs(y - ref)) <= 2e-3
    else:
        y = hip.gemm_f32(a, b, offset)
        ref = oracle.gemm(a, b)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) <= 1e-4
        assert np.all(np.abs(y - ref) <= 1e-3 + 1e-3 * np.abs(ref))
    assert np.isfinite(y).all()


# Narrow N (<= 16) past the skinny kernels: matrix-vector products and a
# few right-hand columns on the narrow kernel. Rows past M in the last
# wavefront, a partial last K step (K = 1000: 125 fp16 / 250 fp32 chunks),
# K shorter than one step, every N from the instance table's ends, M = 1.
GEMM_NARROW = [(4096, 1, 4096), (1000, 3, 1000), (517, 16, 2048), (33, 7, 4096),
               (1, 1, 4096), (2048, 5, 64), (300, 12, 1000), (129, 2, 4096)]


@pytest.mark.parametrize("mnk", GEMM_NARROW)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_gemm_narrow_n(hip, mnk, dtype):
    m, n, k = mnk
    a = oracle.uniform(676 + m, (m, k))
    b = oracle.uniform(677 + n, (k, n))
    if dtype == "f16":
        a, b = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(a, b)
        ref = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b))
        assert np.max(np.abs(y - ref)) <= 2e-3
    else:
        y = hip.gemm_f32(a, b)
        ref = oracle.gemm(a, b)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) <= 1e-4
        assert np.all(np.abs(y - ref) <= 1e-3 + 1e-3 * np.abs(ref))
    assert np.isfinite(y).all()


def test_gemm_narrow_deterministic(hip):
    a = oracle.uniform(678, (1000, 4096))
    b = oracle.uniform(679, (4096, 3))
    first = hip.gemm_f32(a, b)
    for _ in range(3):
        assert np.array_equal(hip.gemm_f32(a, b), first)


@pytest.mark.parametrize("mnk", GEMM_DECODE)
@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_gemm_skinny_wide(hip, mnk, offset, dtype):
    m, n, k = mnk
    a = oracle.uniform(670 + m, (m, k))
    b = oracle.uniform(671 + n, (k, n))
    if dtype == "f16":
        ab, bb = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        fn, ref = hip.lib.operatorlib_gemm_f16, oracle.gemm(oracle.from_f16_bits(ab),
                                                             oracle.from_f16_bits(bb))
        a, b = ab, bb
    else:
        fn, ref = hip.lib.operatorlib_gemm_f32, oracle.gemm(a, b)
    da, db = to_device(a, offset), to_device(b)  # A may be misaligned, B is not
    out = empty((m, n))
    check(fn(ptr(da), ptr(db), ptr(out), m, n, k, stream_handle()), "gemm")
    torch.cuda.synchronize()
    y = out.cpu().numpy().astype(np.float64)
    if dtype == "f16":
        assert np.max(np.abs(y - ref)) <= 2e-3
    else:
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) <= 1e-4
        assert np.all(np.abs(y - ref) <= 1e-3 + 1e-3 * np.abs(ref))
    # deterministic
    check(fn(ptr(da), ptr(db), ptr(out), m, n, k, stream_handle()), "gemm")
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().astype(np.float64), y)


def test_gemm_skinny_deterministic(hip):
    a = oracle.uniform(650, (8, 4096))
    b = oracle.uniform(651, (4096, 2048))
    first = hip.gemm_f32(a, b)
    for _ in range(3):
        assert np.array_equal(hip.gemm_f32(a, b), first)
    # matrix-core variant (fp16, M >= 5)
    ah = oracle.to_f16_bits(oracle.uniform(652, (12, 4096)))
    bh = oracle.to_f16_bits(oracle.uniform(653, (4096, 2048)))
    first = hip.gemm_f16(ah, bh)
    for _ in range(3):
        assert np.array_equal(hip.gemm_f16(ah, bh), first)


# Shapes whose rows are not whole 16-byte chunks or K steps (K or N off the
# chunk multiple, or an unaligned base): the direct-to-LDS kernel reads
# them in place.
GEMM_UNALIGNED = [(1000, 1000, 1000), (1024, 1030, 1024), (1100, 1000, 999), (640, 768, 1800)]


@pytest.mark.parametrize("mnk", GEMM_UNALIGNED)
@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_gemm_unaligned_operands(hip, mnk, offset, dtype):
    m, n, k = mnk
    a = oracle.uniform(620 + m, (m, k))
    b = oracle.uniform(621 + n, (k, n))
    rows = np.unique(np.concatenate([np.arange(40), np.arange(m - 40, m),
                                     np.random.default_rng(m + n).integers(0, m, 48)]))
    if dtype == "f16":
        ab, bb = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(ab, bb, offset)
        ref = oracle.gemm(oracle.from_f16_bits(ab), oracle.from_f16_bits(bb), rows)
        assert np.max(np.abs(y[rows] - ref)) <= 2e-3
    else:
        y = hip.gemm_f32(a, b, offset)
        ref = oracle.gemm(a, b, rows)
        assert np.linalg.norm(y[rows] - ref) / np.linalg.norm(ref) <= 1e-4
    assert np.isfinite(y).all()


@pytest.mark.parametrize("mnk", [(520, 2056, 1024), (1000, 4096, 512), (136, 8192, 256),
                                 (1000, 1028, 520)])
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_gemm_small_grid_tiles(hip, mnk, dtype):
    """Grids too small for 256 x 256 tiles to fill the GPU run on 128 x 128
    tiles: ragged last tile rows / columns (8 or 4 wide), every row checked."""
    m, n, k = mnk
    a = oracle.uniform(660 + m, (m, k))
    b = oracle.uniform(661 + n, (k, n))
    if dtype == "f16":
        a, b = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(a, b)
        ref = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b))
        assert np.max(np.abs(y - ref)) <= 2e-3
    else:
        y = hip.gemm_f32(a, b)
        ref = oracle.gemm(a, b)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) <= 1e-4
    assert np.isfinite(y).all()


@pytest.mark.parametrize("mnk", [(4000, 2600, 1088), (4096, 2560, 64), (1000, 1000, 64),
                                 (520, 2056, 192), (8192, 4096, 192), (4096, 12288, 64),
                                 (4096, 4160, 4096), (4160, 4096, 4032), (4100, 4104, 2048),
                                 (1000, 1000, 32), (600, 1100, 96), (1000, 700, 224),
                                 (520, 2056, 160), (4096, 2560, 96), (4000, 2600, 1056),
                                 (4096, 4096, 4128), (4096, 4160, 4128)])
def test_gemm_f16_step_counts(hip, mnk):
    """fp16 matrix-core tiles over every step-count remainder of their
    loops: 256 x 256 tiles with K % 64 == 0 run 64-deep steps in pairs (odd
    counts, a single step); 128 x 128 tiles (small grids) and 256 x 256
    tiles with K % 64 == 32 run 32-deep steps in fours (1, 2, 3, 5, 6, 7,
    33 and 129 steps); ragged last tile rows and columns; grids of whole
    16 x 16 super-tiles (32 x 16 and 16 x 48 big tiles); and grids one round
    plus 16 or 33 tiles long, whose last round is split along K (16 parts of
    4 steps, 15 uneven parts of 63 steps, 7 parts, and 16 uneven parts of
    32-deep steps)."""
    m, n, k = mnk
    a = oracle.to_f16_bits(oracle.uniform(680 + m, (m, k)))
    b = oracle.to_f16_bits(oracle.uniform(681 + n, (k, n)))
    rows = np.unique(np.concatenate([np.arange(8), np.arange(m - 8, m),
                                     sample_rows(m, 24, 682)]))
    y = hip.gemm_f16(a, b)
    ref = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b), rows)
    assert np.max(np.abs(y[rows] - ref)) <= 2e-3
    assert np.isfinite(y).all()


@pytest.mark.parametrize("mnk", [(4096, 4096, 1056), (4096, 4096, 32), (4096, 4096, 48),
                                 (4096, 4096, 16), (4096, 4100, 256), (4100, 4096, 512),
                                 (4096, 4160, 1024), (4160, 4096, 1040), (520, 2056, 1024),
                                 (1000, 4100, 48), (600, 1100, 16), (1000, 700, 80),
                                 (520, 2052, 112)])
def test_gemm_f32_step_counts(hip, mnk):
    """fp32 direct-to-LDS tiles over every step-count remainder of their
    loops: 256 x 256 tiles with K % 32 == 0 run 32-deep steps in pairs (33
    steps, a single step); with K % 32 == 16, 16-deep steps in fours (3
    steps, 1 step); a ragged last tile column of one 4-column chunk and a
    ragged last tile row; grids one round plus 16 tiles long whose last
    round is split along K (2 parts, 4 parts of 8 steps, 4 uneven parts of
    16-deep steps); 128 x 128 tiles on small grids (64, 3, 1, 5 and 7
    steps, N off a multiple of 8)."""
    m, n, k = mnk
    a = oracle.uniform(690 + m, (m, k))
    b = oracle.uniform(691 + n, (k, n))
    rows = np.unique(np.concatenate([np.arange(8), np.arange(m - 8, m),
                                     sample_rows(m, 24, 692)]))
    y = hip.gemm_f32(a, b)
    ref = oracle.gemm(a, b, rows)
    assert np.linalg.norm(y[rows] - ref) / np.linalg.norm(ref) <= 1e-4
    assert np.all(np.abs(y[rows] - ref) <= 1e-3 + 1e-3 * np.abs(ref))
    assert np.isfinite(y).all()


@pytest.mark.parametrize("mnk", [(65, 4096, 4096), (100, 4096, 4096), (128, 1000, 4096),
                                 (96, 4100, 2048), (256, 4096, 512), (200, 3000, 2048),
                                 (48, 4096, 4096)])
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_gemm_small_m_split_k(hip, mnk, dtype):
    """M past the skinny kernels (32 rows fp16, 64 fp32) on a grid of fewer
    128 x 128 tiles than CUs: every tile is split along K (16 parts at K =
    4096, 2 at K = 512 where the depth limit binds, 10 uneven parts on 48
    tiles) and the parts summed; ragged N (1000, 4100); M = 48 fp16. Every
    row checked."""
    m, n, k = mnk
    a = oracle.uniform(650 + m, (m, k))
    b = oracle.uniform(651 + n, (k, n))
    if dtype == "f16":
        a, b = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(a, b)
        ref = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b))
        assert np.max(np.abs(y - ref)) <= 2e-3
    else:
        y = hip.gemm_f32(a, b)
        ref = oracle.gemm(a, b)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) <= 1e-4
    assert np.isfinite(y).all()


@pytest.mark.parametrize("mnk", [(4097, 4095, 4093), (4352, 4100, 999)])
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_gemm_unaligned_split_tail(hip, mnk, dtype):
    """Unaligned operands on a grid one round plus 16 (33) 256 x 256 tiles
    long: the last round is split along K (16 parts; 3 parts), and the
    last part repairs the partly filled last K step."""
    m, n, k = mnk
    a = oracle.uniform(640 + m, (m, k))
    b = oracle.uniform(641 + n, (k, n))
    rows = tile_row_rows(m, 642)
    if dtype == "f16":
        a, b = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(a, b)
        ref = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b), rows)
        assert np.max(np.abs(y[rows] - ref)) <= 2e-3
    else:
        y = hip.gemm_f32(a, b)
        ref = oracle.gemm(a, b, rows)
        assert np.linalg.norm(y[rows] - ref) / np.linalg.norm(ref) <= 1e-4
    assert np.isfinite(y).all()


def test_gemm_split_then_smaller(hip):
    """The arena is reused: a call with split partials followed by a smaller
    one and a larger one must all be right."""
    for m, n, k in [(1200, 1100, 1001), (700, 800, 1999), (1500, 1500, 1500)]:
        a = oracle.uniform(630 + m, (m, k))
        b = oracle.uniform(631 + n, (k, n))
        ab, bb = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(ab, bb)
        rows = np.array([0, 1, m // 2, m - 2, m - 1])
        ref = oracle.gemm(oracle.from_f16_bits(ab), oracle.from_f16_bits(bb), rows)
        assert np.max(np.abs(y[rows] - ref)) <= 2e-3


# Shapes off every rule of the skinny and narrow kernels (odd N, odd K),
# K shorter than one K step, single rows and columns: all run the
# direct-to-LDS kernel in place, whose first step is the partly filled
# last one.
GEMM_ODD = [(1, 1001, 333), (3, 7, 5), (17, 9, 1), (100, 5, 33), (129, 257, 63),
            (300, 301, 7), (65, 1000, 4095), (257, 255, 97)]


@pytest.mark.parametrize("mnk", GEMM_ODD)
@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_gemm_odd_shapes(hip, mnk, offset, dtype):
    m, n, k = mnk
    a = oracle.uniform(690 + m, (m, k))
    b = oracle.uniform(691 + n, (k, n))
    if dtype == "f16":
        ab, bb = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(ab, bb, offset)
        ref = oracle.gemm(oracle.from_f16_bits(ab), oracle.from_f16_bits(bb))
        assert np.max(np.abs(y - ref)) <= 2e-3
    else:
        y = hip.gemm_f32(a, b, offset)
        ref = oracle.gemm(a, b)
        assert np.linalg.norm(y - ref) / np.linalg.norm(ref) <= 1e-4
        assert np.all(np.abs(y - ref) <= 1e-3 + 1e-3 * np.abs(ref))


# Grids of 256 x 256 tiles whose last K step is partly filled, on both the
# 64-deep (fp32: 32) and the half-deep stages, with odd N; and medium grids.
GEMM_PARTIAL_STEP = [(4096, 4095, 3999), (4096, 4095, 4001), (4095, 4097, 3983),
                     (2000, 1999, 1001)]


@pytest.mark.parametrize("mnk", GEMM_PARTIAL_STEP)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_gemm_partial_last_step(hip, mnk, dtype):
    m, n, k = mnk
    a = oracle.uniform(700 + k, (m, k))
    b = oracle.uniform(701 + n, (k, n))
    rows = tile_row_rows(m, 702)
    if dtype == "f16":
        a, b = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(a, b)
        ref = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b), rows)
        assert np.max(np.abs(y[rows] - ref)) <= 2e-3
    else:
        y = hip.gemm_f32(a, b)
        ref = oracle.gemm(a, b, rows)
        assert np.linalg.norm(y[rows] - ref) / np.linalg.norm(ref) <= 1e-4
    assert np.isfinite(y).all()


# Large fp16 products whose A rows (odd K, or a base off 4 bytes), B rows
# (odd N) or both are not 4-byte aligned copy operands into chunk-padded
# rows first: A alone (odd K), B alone (odd N), A alone with both off at
# mid size (base offset), both with K padded too (6000 x 6001 x 6003).
@pytest.mark.parametrize("mnk_off", [(4096, 8192, 4099, 0), (4096, 8191, 4100, 0),
                                     (4096, 4096, 4096, 1), (6000, 6001, 6003, 0)])
def test_gemm_f16_padded_rows(hip, mnk_off):
    m, n, k, offset = mnk_off
    a = oracle.to_f16_bits(oracle.uniform(720 + k, (m, k)))
    b = oracle.to_f16_bits(oracle.uniform(721 + n, (k, n)))
    rows = tile_row_rows(m, 722)
    y = hip.gemm_f16(a, b, offset)
    ref = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b), rows)
    assert np.max(np.abs(y[rows] - ref)) <= 2e-3
    assert np.isfinite(y).all()


@pytest.mark.parametrize("mnk", [(300, 301, 999), (1000, 999, 1001), (4096, 4095, 4095),
                                 (5, 1001, 77)])
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_gemm_reads_nothing_past_k_or_the_operands(hip, mnk, dtype):
    """A and B start NaN-filled allocations, and a few rows of A start with
    NaN. The copies of a row's last K step run into the next row (and past
    the end of A and B for the last rows): rows whose own elements are
    finite must come out finite and equal to the oracle, the NaN rows NaN,
    and the last elements of A and B (read through a partly out-of-range
    dword with fp16) must count."""
    m, n, k = mnk
    rng = np.random.default_rng(m + 7 * n + k)
    a = oracle.uniform(710 + m, (m, k))
    b = oracle.uniform(711 + n, (k, n))
    a[m - 1, k - 1] = 64.0  # exact in fp16; a lost end element shows at once
    b[k - 1, n - 1] = -64.0
    nan_rows = np.unique(rng.integers(1, m, 3)) if m > 2 else np.array([], dtype=np.int64)
    a[nan_rows, 0] = np.nan
    if dtype == "f16":
        a_dev, b_dev = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        torch_dtype, fn = torch.float16, hip.lib.operatorlib_gemm_f16
        a_ref, b_ref = oracle.from_f16_bits(a_dev), oracle.from_f16_bits(b_dev)
    else:
        a_dev, b_dev, a_ref, b_ref = a, b, a, b
        torch_dtype, fn = torch.float32, hip.lib.operatorlib_gemm_f32
    bufs = []
    for host in (a_dev, b_dev):
        buf = torch.full((host.size + 4096,), float("nan"), dtype=torch_dtype, device="cuda")
        src = torch.from_numpy(host.view(np.float16) if dtype == "f16" else host).reshape(-1)
        buf[:host.size].copy_(src.to("cuda"))
        bufs.append(buf)
    out = empty((m, n))
    check(fn(ptr(bufs[0]), ptr(bufs[1]), ptr(out), m, n, k, stream_handle()), "gemm")
    torch.cuda.synchronize()
    y = out.cpu().numpy().astype(np.float64)
    finite_rows = np.setdiff1d(np.arange(m), nan_rows)
    rows = np.unique(np.concatenate([finite_rows[:4], finite_rows[-4:], nan_rows - 1,
                                     rng.choice(finite_rows, min(24, finite_rows.size),
                                                replace=False)]))
    rows = np.setdiff1d(rows, nan_rows)
    ref = oracle.gemm(np.nan_to_num(a_ref[rows], nan=0.0), b_ref)
    assert np.isfinite(y[finite_rows]).all()
    if dtype == "f16":
        assert np.max(np.abs(y[rows] - ref)) <= 2e-3
    else:
        assert np.linalg.norm(y[rows] - ref) / np.linalg.norm(ref) <= 1e-4
    assert np.isnan(y[nan_rows]).all()


def test_gemm_pins(hip):
    pins.pin_gemm(hip.gemm_f32)
    f16 = lambda a, b: hip.gemm_f16(oracle.to_f16_bits(a), oracle.to_f16_bits(b))
    pins.pin_gemm(f16)  # every pin input is exactly representable in fp16


def tile_row_rows(size: int, seed: int, tile: int = 256) -> np.ndarray:
    """A seeded row inside every `tile`-row band of C, both rows at every band
    boundary, and the first and last rows: every 256 x 256 tile row of the
    GEMM grid (and, since rows are compared whole, every tile) is checked."""
    rng = np.random.default_rng(seed)
    rows = {0, size - 1}
    for t0 in range(0, size, tile):
        rows.add(int(t0 + rng.integers(0, min(tile, size - t0))))
        if t0 > 0:
            rows.update({t0 - 1, t0})
    return np.array(sorted(rows), dtype=np.int32)


@pytest.mark.parametrize("dtype,size", [("f32", 4096), ("f32", 4095), ("f16", 4096),
                                        ("f16", 4095), ("f16", 8192)])
def test_gemm_baseline_sizes(hip, dtype, size):
    a = oracle.uniform(800 + size, (size, size))
    b = oracle.uniform(801 + size, (size, size))
    rows = tile_row_rows(size, 802)
    if dtype == "f16":
        a, b = oracle.to_f16_bits(a), oracle.to_f16_bits(b)
        y = hip.gemm_f16(a, b)
        ref = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b), rows)
        assert np.max(np.abs(y[rows] - ref)) <= 2e-3
    else:
        y = hip.gemm_f32(a, b)
        ref = oracle.gemm(a, b, rows)
        assert np.linalg.norm(y[rows] - ref) / np.linalg.norm(ref) <= 1e-4
    assert np.isfinite(y).all()


@pytest.mark.parametrize("m,n,k", [(8191, 8191, 8191), (8192, 8190, 8192)])
def test_gemm_f16_streaming_c_odd_rows(hip, m, n, k):
    # Four rounds of 256 x 256 tiles with A + B past 192 MiB: C is stored
    # non-temporally through the LDS-staged epilogue, here with C rows off
    # 16-byte alignment (N = 8191, 8190), A / B rows at a 2-byte phase
    # (8191: the edge instance) and partial edge tiles on the per-float path.
    rng = np.random.default_rng(811)
    a = oracle.to_f16_bits(oracle.uniform(812, (m, k)))
    b = oracle.to_f16_bits(oracle.uniform(813, (k, n)))
    bands = np.arange(0, m, 256)
    picks = np.minimum(bands + rng.integers(0, 256, bands.size), m - 1)
    rows = np.unique(np.concatenate([[0, 1, m - 2, m - 1], picks])).astype(np.int32)
    y = hip.gemm_f16(a, b)
    ref = oracle.gemm(oracle.from_f16_bits(a), oracle.from_f16_bits(b), rows)
    assert np.max(np.abs(y[rows] - ref)) <= 2e-3
    assert np.isfinite(y).all()


# --------------------------------------------------------------------- attention

# (S, D, causal, extreme): tests/attention_smoke.cu:168-173, edge shapes, and
# shapes on this library's fp16 global->LDS path (D 64/128, aligned tensors:
# offset 0).
ATTN_SMALL = [(32, 64, False, False), (32, 128, True, False), (37, 71, True, True),
              (1, 1, False, False), (5, 16, True, False), (129, 32, True, False),
              (200, 96, False, False), (257, 128, True, False), (64, 40, False, False),
              (128, 128, True, False), (256, 64, True, False), (384, 64, False, False),
              (512, 128, False, True), (256, 128, True, True)]


def _attn_inputs(s, d, extreme, seed, heads=2):
    r = 20.0 if extreme else 1.0
    q = oracle.uniform(seed, (1, heads, s, d), -r, r)
    k = oracle.uniform(seed + 1, (1, heads, s, d), -r, r)
    v = oracle.uniform(seed + 2, (1, heads, s, d))
    return q, k, v


@pytest.mark.parametrize("s,d,causal,extreme", ATTN_SMALL)
@pytest.mark.parametrize("offset", [0, 1])
def test_attention_f32_small(hip, s, d, causal, extreme, offset):
    q, k, v = _attn_inputs(s, d, extreme, 900 + s + d)
    ref = oracle.attention(q, k, v, causal)
    y = hip.attention(q, k, v, causal, offset)
    assert np.all(np.abs(y - ref) <= 1e-4 + 1e-4 * np.abs(ref))


@pytest.mark.parametrize("s,d,causal,extreme", ATTN_SMALL)
@pytest.mark.parametrize("offset", [0, 1])
def test_attention_f16_small(hip, s, d, causal, extreme, offset):
    q, k, v = _attn_inputs(s, d, extreme, 950 + s + d)
    qb, kb, vb = (oracle.to_f16_bits(t) for t in (q, k, v))
    ref = oracle.attention(*(oracle.from_f16_bits(t) for t in (qb, kb, vb)), causal)
    y = hip.attention(qb, kb, vb, causal, offset)
    # extreme (+-20) inputs use the reference's own 2e-2 bound
    # (tests/attention_smoke.cu:154); the rest the 2e-3 contract
    assert np.max(np.abs(y - ref)) <= (2e-2 if extreme else 2e-3)


@pytest.mark.parametrize("heads,s,d,causal", [
    # 64-row blocks, keys split: D 128 up to 128 query blocks (of 128 rows),
    # D 64 up to 384 (512 causal)
    (1, 384, 128, True), (3, 384, 64, True), (9, 256, 128, False), (5, 128, 64, True),
    (128, 128, 128, True), (43, 384, 64, False), (168, 384, 64, True),
    (256, 256, 64, True),
    # D 128, 128-row blocks, keys split (<= 256 blocks, < 512 causal)
    (50, 384, 128, False), (100, 384, 128, True), (64, 512, 128, False),
    # 128-row blocks, keys not split
    (512, 128, 128, False), (86, 384, 128, False), (129, 384, 64, False),
    (171, 384, 64, True)])
def test_attention_f16_fast_path_covers_every_block(hip, heads, s, d, causal):
    # (heads x query blocks) not a multiple of 8: the work items are split
    # over 8 XCD ranges and the grid is padded; every row must be written.
    # Small grids run 64-row blocks; mid-size D 128 grids (up to 256 blocks,
    # under 512 causal) split each block's keys between two wavefront groups of
    # the workgroup; larger ones do not.
    q, k, v = _attn_inputs(s, d, False, 970 + heads + s, heads=heads)
    qb, kb, vb = (oracle.to_f16_bits(t) for t in (q, k, v))
    ref = oracle.attention(*(oracle.from_f16_bits(t) for t in (qb, kb, vb)), causal)
    y = hip.attention(qb, kb, vb, causal)
    assert np.isfinite(y).all()
    assert np.max(np.abs(y - ref)) <= 2e-3


@pytest.mark.parametrize("heads,s,d,causal", [
    # 64-row blocks (four key groups at D 128, two at D 64)
    (1, 1, 128, False), (2, 33, 128, True), (3, 100, 128, False), (1, 1000, 128, True),
    (12, 1000, 128, False), (3, 65, 64, True), (5, 1000, 64, False),
    # D 128, 128-row blocks, keys split between two groups
    (50, 300, 128, False), (100, 300, 128, True),
    # 128-row blocks, keys not split
    (260, 200, 128, False), (171, 383, 64, True), (129, 383, 64, False)])
def test_attention_f16_fast_path_ragged_sequence(hip, heads, s, d, causal):
    # S not a multiple of the query block: the last block's rows past S are
    # computed from row S - 1 of Q and not stored, keys past S read zeros
    # and are masked; every row up to S must be written and match the oracle.
    q, k, v = _attn_inputs(s, d, False, 990 + heads + s, heads=heads)
    qb, kb, vb = (oracle.to_f16_bits(t) for t in (q, k, v))
    ref = oracle.attention(*(oracle.from_f16_bits(t) for t in (qb, kb, vb)), causal)
    y = hip.attention(qb, kb, vb, causal)
    assert np.isfinite(y).all()
    assert np.max(np.abs(y - ref)) <= 2e-3


@pytest.mark.parametrize("heads,s,d,causal", [
    # 64-row blocks, keys split between two groups (D 128 up to 128 blocks,
    # D 64 up to 384 / 512 causal), several tiles per group
    (2, 333, 128, True), (3, 100, 128, False), (4, 1000, 128, False), (2, 2000, 128, True),
    (3, 65, 64, True), (100, 100, 64, False),
    # D 128, 128-row blocks, keys split (<= 256 blocks, < 512 causal)
    (200, 100, 128, False), (300, 100, 128, True),
    # 128-row blocks, keys not split
    (260, 100, 128, False), (520, 100, 128, True), (390, 100, 64, False),
    (520, 100, 64, True)])
def test_attention_f32_fast_path(hip, heads, s, d, causal):
    """fp32 on the direct-to-LDS kernel (D 64 / 128, aligned tensors): every
    instance, ragged sequence lengths (keys past S read zeros and are
    masked, rows past S are not stored), every row against the oracle."""
    q, k, v = _attn_inputs(s, d, False, 1010 + heads + s, heads=heads)
    ref = oracle.attention(q, k, v, causal)
    y = hip.attention(q, k, v, causal)
    assert np.isfinite(y).all()
    assert np.all(np.abs(y - ref) <= 1e-4 + 1e-4 * np.abs(ref))


# (heads, S, D, causal) on every fp16 fast-path instance with S ragged:
# D 128 64-row blocks / 128-row blocks with keys split / unsplit, D 64
# 64-row blocks / 128-row blocks.
POISON_CASES = [(1, 300, 128, False), (2, 1000, 128, True), (50, 300, 128, False),
                (20, 1000, 128, True), (100, 300, 128, False), (70, 1000, 128, True),
                (1, 1000, 64, True), (3, 300, 64, False), (200, 300, 64, True),
                (60, 1000, 64, False),
                # head dims padded to the 64 / 128 layouts (dims past D read zeros)
                (1, 300, 96, False), (20, 1000, 80, True), (100, 300, 96, False),
                (3, 300, 48, True), (200, 300, 32, False)]


# Head dims other than 64 and 128 (whole 16-byte chunks) run the 64 / 128
# fast-path instances with the dims past D zero in Q, K and V; only D
# columns of O are stored. (heads, S, D, causal) over 64-row blocks, split
# keys and unsplit grids.
PADDED_CASES = [(2, 333, 96, False), (12, 1000, 80, True), (100, 300, 96, True),
                (300, 129, 120, False), (4, 200, 8, False), (50, 300, 16, True),
                (200, 300, 40, False), (520, 100, 56, True)]


# Short sequences (S <= 64) on more than 128 heads: 64-row blocks of two
# wavefronts on 32-key tiles, both layouts, padded dims included.
@pytest.mark.parametrize("heads,s,d,causal", [(200, 16, 128, False), (300, 64, 64, True),
                                              (150, 1, 128, False), (140, 33, 96, True),
                                              (260, 7, 40, False), (129, 64, 128, True)])
def test_attention_f16_short_sequences(hip, heads, s, d, causal):
    q, k, v = _attn_inputs(s, d, False, 1400 + heads + s, heads=heads)
    qb, kb, vb = (oracle.to_f16_bits(t) for t in (q, k, v))
    ref = oracle.attention(*(oracle.from_f16_bits(t) for t in (qb, kb, vb)), causal)
    y = hip.attention(qb, kb, vb, causal)
    assert np.isfinite(y).all()
    assert np.max(np.abs(y - ref)) <= 2e-3


@pytest.mark.parametrize("heads,s,d,causal", PADDED_CASES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_attention_padded_head_dims(lib, heads, s, d, causal, dtype):
    q, k, v = _attn_inputs(s, d, False, 1300 + heads + d, heads=heads)
    n = heads * s * d
    guard = 64 * d
    out_flat = torch.full((n + guard,), float("nan"), dtype=torch.float32, device="cuda")
    if dtype == "f16":
        bits = [oracle.to_f16_bits(t) for t in (q, k, v)]
        dq, dk, dv = (to_device(b) for b in bits)
        ref_in = [oracle.from_f16_bits(b) for b in bits]
        fn, tol = lib.operatorlib_attention_f16, None
    else:
        dq, dk, dv = (to_device(t) for t in (q, k, v))
        ref_in = [q, k, v]
        fn, tol = lib.operatorlib_attention_f32, 1e-4
    check(fn(ptr(dq), ptr(dk), ptr(dv), ptr(out_flat), 1, heads, s, d, int(causal),
             stream_handle()), "attention")
    torch.cuda.synchronize()
    flat = out_flat.cpu().numpy().astype(np.float64)
    assert np.isnan(flat[n:]).all()  # nothing stored past the output
    y = flat[:n].reshape(heads, s, d)
    rng = np.random.default_rng(1301)
    hs = np.concatenate([np.full(s, heads - 1), rng.integers(0, heads, 256)]).astype(np.int32)
    rs = np.concatenate([np.arange(s), rng.integers(0, s, 256)]).astype(np.int32)
    ref = oracle.attention(*ref_in, causal, hs, rs)
    assert np.isfinite(y).all()
    if tol is None:
        assert np.max(np.abs(y[hs, rs] - ref)) <= 2e-3
    else:
        assert np.all(np.abs(y[hs, rs] - ref) <= tol + tol * np.abs(ref))


@pytest.mark.parametrize("heads,s,d,causal", POISON_CASES)
def test_attention_f16_reads_no_key_past_the_sequence(lib, heads, s, d, causal):
    # Q, K and V end one 64-key tile before the end of an allocation whose
    # tail holds NaN. The last key tile of every head runs past S; its keys
    # from S on must read zeros (a read of the next head's rows or of the
    # NaN tail would turn P.V into NaN, since masked p = 0 times NaN is NaN).
    q, k, v = _attn_inputs(s, d, False, 1100 + heads + s, heads=heads)
    bits = [oracle.to_f16_bits(t) for t in (q, k, v)]
    tail = 64 * d

    def poisoned(b):
        flat = torch.full((b.size + tail,), float("nan"), dtype=torch.float16, device="cuda")
        flat[:b.size].copy_(torch.from_numpy(b.reshape(-1).view(np.float16)).to("cuda"))
        return flat

    dq, dk, dv = (poisoned(b) for b in bits)
    out = empty((1, heads, s, d))
    check(lib.operatorlib_attention_f16(ptr(dq), ptr(dk), ptr(dv), ptr(out), 1, heads, s,
                                        d, int(causal), stream_handle()), "attention_f16")
    torch.cuda.synchronize()
    y = out.cpu().numpy().astype(np.float64).reshape(heads, s, d)
    assert np.isfinite(y).all()
    # the last head in full, plus seeded rows of the others
    rng = np.random.default_rng(1101)
    hs = np.concatenate([np.full(s, heads - 1), rng.integers(0, heads, 256)]).astype(np.int32)
    rs = np.concatenate([np.arange(s), rng.integers(0, s, 256)]).astype(np.int32)
    ref = oracle.attention(*(oracle.from_f16_bits(b) for b in bits), causal, hs, rs)
    assert np.max(np.abs(y[hs, rs] - ref)) <= 2e-3


@pytest.mark.parametrize("heads,s,d,causal", POISON_CASES)
def test_attention_f32_reads_no_key_past_the_sequence(lib, heads, s, d, causal):
    # The same NaN tail after fp32 Q, K and V, on the fp32 fast-path
    # instances (the cases span their 64-row, key-split and unsplit grids).
    q, k, v = _attn_inputs(s, d, False, 1200 + heads + s, heads=heads)
    tail = 64 * d

    def poisoned(a):
        flat = torch.full((a.size + tail,), float("nan"), dtype=torch.float32, device="cuda")
        host = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
        flat[:a.size].copy_(torch.from_numpy(host).to("cuda"))
        return flat

    dq, dk, dv = (poisoned(a) for a in (q, k, v))
    out = empty((1, heads, s, d))
    check(lib.operatorlib_attention_f32(ptr(dq), ptr(dk), ptr(dv), ptr(out), 1, heads, s,
                                        d, int(causal), stream_handle()), "attention_f32")
    torch.cuda.synchronize()
    y = out.cpu().numpy().astype(np.float64).reshape(heads, s, d)
    assert np.isfinite(y).all()
    rng = np.random.default_rng(1201)
    hs = np.concatenate([np.full(s, heads - 1), rng.integers(0, heads, 256)]).astype(np.int32)
    rs = np.concatenate([np.arange(s), rng.integers(0, s, 256)]).astype(np.int32)
    ref = oracle.attention(q, k, v, causal, hs, rs)
    assert np.all(np.abs(y[hs, rs] - ref) <= 1e-4 + 1e-4 * np.abs(ref))


def test_attention_pins(hip):
    pins.pin_attention(hip.attention, tol=2e-6)
    f16 = lambda q, k, v, c: hip.attention(*(oracle.to_f16_bits(t) for t in (q, k, v)), c)
    pins.pin_attention(f16, tol=1e-2)


@pytest.mark.parametrize("b,h,s,causal", [(1, 12, 1024, False), (1, 12, 1024, True),
                                          (4, 32, 8192, True)])
def test_attention_f16_baseline(hip, b, h, s, causal):
    d = 128
    q, k, v = (oracle.to_f16_bits(oracle.normal(1000 + i, (b, h, s, d))) for i in range(3))
    y = hip.attention(q, k, v, causal)
    qf, kf, vf = (oracle.from_f16_bits(t) for t in (q, k, v))
    if s <= 1024:  # every row
        ref = oracle.attention(qf, kf, vf, causal)
        assert np.max(np.abs(y - ref)) <= 2e-3
        return
    # One seeded row in every (head, 128-row query block) work item of the
    # fast path, plus in every head the first and last rows and both rows at
    # the edges of the first query block's diagonal tile (SURVEY-scale
    # sample: 128 x 64 + 128 x 8 = 9216 rows).
    rng = np.random.default_rng(1001)
    blocks = s // 128
    heads = np.repeat(np.arange(b * h, dtype=np.int32), blocks)
    rws = (np.tile(np.arange(blocks, dtype=np.int32) * 128, b * h) +
           rng.integers(0, 128, b * h * blocks).astype(np.int32))
    edges = np.array([0, 1, 63, 64, 127, 128, s - 2, s - 1], np.int32)
    heads = np.concatenate([heads, np.repeat(np.arange(b * h, dtype=np.int32), edges.size)])
    rws = np.concatenate([rws, np.tile(edges, b * h)])
    ref = oracle.attention(qf, kf, vf, causal, heads, rws)
    got = y.reshape(b * h, s, d)[heads, rws]
    assert np.max(np.abs(got - ref)) <= 2e-3
    assert np.isfinite(y).all()
