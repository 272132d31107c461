"""Per-op parity of libsfg_hip.so against the CPU oracle (GPU only).

Tolerances: integer / index outputs bit-exact; fp32 paths 1e-4 relative
(max|got-ref| / max|ref|); bf16 paths 2e-2; int8-weight paths 1e-2.
Integer-valued operands make GEMM results exact in fp32, which pins the MFMA
operand/accumulator lane layouts bit for bit.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from schedforge_amd import _abi
from schedforge_amd._abi import BF16, EPI_GLU_SILU_UP, EPI_NONE, EPI_RESIDUAL, EPI_SWIGLU, F32, I8

from _helpers import bf16_dev, bf16_host, dev, host, stream, tile_nk

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def lib():
    return _abi.load()


def _sync():
    torch.cuda.synchronize()


# ------------------------------------------------------------------ RMSNorm
@pytest.mark.parametrize("rows,width", [(16, 2048), (7, 250), (128, 256)])
def test_rmsnorm_f32_matches_oracle(lib, rows, width):
    x = oracle.normal(11, 0, (rows, width))
    w = oracle.normal(11, 1, (width,), 0.5, 1.0)
    y = torch.empty((rows, width), dtype=torch.float32, device="cuda")
    _abi.check(lib.sfg_hip_rmsnorm_v1(dev(x).data_ptr(), dev(w).data_ptr(), y.data_ptr(), F32,
                                      rows, width, ctypes.c_float(1e-5), stream()))
    ref = oracle.rms_norm(x, w, 1e-5)
    got = host(y)
    # double accumulation + correctly rounded sqrt/div: bit-exact except for a
    # rare last-bit difference of the double sum's rounding order.
    assert np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)) < 2.5e-7


def test_rmsnorm_constant_row_closed_form(lib):
    c, eps, width = 0.75, 1e-6, 1024
    x = np.full((3, width), c, np.float32)
    w = np.linspace(0.5, 1.5, width).astype(np.float32)
    y = torch.empty((3, width), dtype=torch.float32, device="cuda")
    _abi.check(lib.sfg_hip_rmsnorm_v1(dev(x).data_ptr(), dev(w).data_ptr(), y.data_ptr(), F32, 3,
                                      width, ctypes.c_float(eps), stream()))
    expect = c * w / np.sqrt(c * c + eps)
    np.testing.assert_allclose(host(y), np.broadcast_to(expect, (3, width)), rtol=3e-7)


def test_rmsnorm_bf16_output_is_rne_of_f32(lib):
    x = oracle.normal(12, 0, (16, 2048))
    w = np.ones(2048, np.float32)
    y32 = torch.empty((16, 2048), dtype=torch.float32, device="cuda")
    y16 = torch.empty((16, 2048), dtype=torch.int16, device="cuda")
    xd, wd = dev(x), dev(w)
    _abi.check(lib.sfg_hip_rmsnorm_v1(xd.data_ptr(), wd.data_ptr(), y32.data_ptr(), F32, 16, 2048,
                                      ctypes.c_float(1e-5), stream()))
    _abi.check(lib.sfg_hip_rmsnorm_v1(xd.data_ptr(), wd.data_ptr(), y16.data_ptr(), BF16, 16, 2048,
                                      ctypes.c_float(1e-5), stream()))
    np.testing.assert_array_equal(host(y16).view(np.uint16), oracle.to_bf16_bits(host(y32)))


# ------------------------------------------------------------------ GEMM
def _gemm(lib, a_dev, a_dtype, b_dev, b_dtype, m, n, k, epi, c_dtype=F32, scales=None,
          residual=None, layout=0, tile=0, workspace=True):
    glu = epi in (EPI_SWIGLU, EPI_GLU_SILU_UP)
    c = torch.empty((m, n), dtype=torch.float32 if c_dtype == F32 else torch.int16, device="cuda")
    args = _abi.GemmArgs()
    args.a, args.a_dtype, args.lda = a_dev.data_ptr(), a_dtype, k
    args.b, args.b_dtype, args.ldb = b_dev.data_ptr(), b_dtype, k
    args.b_scales = scales.data_ptr() if scales is not None else None
    args.c, args.c_dtype, args.ldc = c.data_ptr(), c_dtype, n
    args.residual = residual.data_ptr() if residual is not None else None
    args.ldr = n
    args.m, args.n, args.k, args.epilogue = m, n, k, epi
    args.b_layout = layout
    args.tile = tile
    if workspace:
        wsb = lib.sfg_hip_gemm_workspace_v1(m, n, k)
        ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device="cuda")
        _abi.check(lib.sfg_hip_gemm_v1(ctypes.byref(args), ws.data_ptr(), ws.numel(), stream()))
    else:
        _abi.check(lib.sfg_hip_gemm_v1(ctypes.byref(args), None, 0, stream()))
    _sync()
    return c


@pytest.mark.parametrize("tile", list(range(1, _abi.TILE_COUNT)))
@pytest.mark.parametrize("m,n,k,epi", [(1024, 512, 256, EPI_NONE), (1300, 768, 320, EPI_RESIDUAL),
                                       (2048, 512, 192, EPI_SWIGLU)])
def test_gemm_every_tile_policy_exact(lib, tile, m, n, k, epi):
    """Each sfg_gemm_tile of the direct-to-LDS kernel, on small-integer
    operands (every partial sum exact in fp32): a wrong fragment, swizzle or
    edge mask shows as a difference.  Ragged M / N exercise the tile edges."""
    rng = np.random.default_rng(tile * 131 + m)
    glu = epi == EPI_SWIGLU
    a = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
    b = rng.integers(-3, 4, size=((2 * n) if glu else n, k)).astype(np.float32)
    res = rng.integers(-5, 6, size=(m, n)).astype(np.float32)
    c = _gemm(lib, bf16_dev(a), BF16, bf16_dev(b), BF16, m, n, k, epi,
              residual=dev(res) if epi == EPI_RESIDUAL else None, tile=tile)
    acc = a.astype(np.float64) @ b.T.astype(np.float64)
    if glu:
        np.testing.assert_allclose(host(c), _ref_epilogue(acc, epi, n), rtol=1e-5, atol=1e-5)
    else:
        np.testing.assert_array_equal(host(c), _ref_epilogue(acc, epi, n, res).astype(np.float32))


@pytest.mark.parametrize("tile,k", [(_abi.TILE_256x256_PP, 64), (_abi.TILE_256x256_V, 64),
                                    (_abi.TILE_256x256_V, 128)])
@pytest.mark.parametrize("epi", [EPI_NONE, EPI_RESIDUAL, EPI_SWIGLU, EPI_GLU_SILU_UP])
def test_gemm_many_tiles_exact(lib, epi, tile, k):
    """More 256 x 256 tiles than the CUs hold at once, ragged in both
    directions, K shorter than the LDS ring (ping-pong: two 32-k slabs in a
    four-stage ring; register prefetch: one or two 64-k slabs, fewer than the
    three it keeps in flight): small-integer operands keep every sum exact, so
    a tile mapped twice, skipped, or read from a stale stage shows as a
    difference."""
    m, n = 4400, 4360
    glu = epi in (EPI_SWIGLU, EPI_GLU_SILU_UP)
    rng = np.random.default_rng(977 + epi + k)
    a = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
    b = rng.integers(-3, 4, size=((2 * n) if glu else n, k)).astype(np.float32)
    res = rng.integers(-5, 6, size=(m, n)).astype(np.float32)
    c = _gemm(lib, bf16_dev(a), BF16, bf16_dev(b), BF16, m, n, k, epi,
              residual=dev(res) if epi == EPI_RESIDUAL else None, tile=tile)
    acc = a.astype(np.float64) @ b.T.astype(np.float64)
    if glu:
        np.testing.assert_allclose(host(c), _ref_epilogue(acc, epi, n), rtol=1e-5, atol=1e-5)
    else:
        np.testing.assert_array_equal(host(c), _ref_epilogue(acc, epi, n, res).astype(np.float32))


def test_gemm_rejects_unknown_tile(lib):
    a = bf16_dev(np.ones((1024, 64), np.float32))
    with pytest.raises(ValueError):
        _gemm(lib, a, BF16, a, BF16, 1024, 1024, 64, EPI_NONE, tile=_abi.TILE_COUNT)


def _ref_epilogue(acc, epi, n, residual=None):
    if epi == EPI_NONE:
        return acc
    if epi == EPI_RESIDUAL:
        return acc + residual
    g, u = acc[:, :n], acc[:, n:]
    # exponent clamped: large-magnitude negatives give silu = -0 without overflow
    if epi == EPI_SWIGLU:
        return g / (1 + np.exp(np.minimum(-g, 700.0))) * u
    return g * (u / (1 + np.exp(np.minimum(-u, 700.0))))


@pytest.mark.parametrize("m,n,k", [(16, 3072, 2048), (16, 512, 5632), (64, 1024, 512), (5, 256, 384),
                                   (256, 512, 256), (512, 1024, 512), (300, 256, 128),
                                   (1024, 512, 256), (1300, 256, 192), (2048, 1024, 1024),
                                   (1536, 768, 320), (1100, 384, 64)])
def test_gemm_bf16_integer_operands_exact(lib, m, n, k):
    """Small-integer operands: every product and partial sum is exact in fp32,
    so any lane-layout or indexing mistake shows as a nonzero difference."""
    rng = np.random.default_rng(m * 7 + n)
    a = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
    b = rng.integers(-3, 4, size=(n, k)).astype(np.float32)
    c = _gemm(lib, bf16_dev(a), BF16, bf16_dev(b), BF16, m, n, k, EPI_NONE)
    np.testing.assert_array_equal(host(c), a @ b.T)


@pytest.mark.parametrize("m,n,k", [(16, 2048, 2048), (9, 256, 8192), (64, 512, 1024), (200, 512, 256),
                                   (1100, 256, 128)])
def test_gemm_int8_integer_operands_exact(lib, m, n, k):
    rng = np.random.default_rng(m + n + k)
    a = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
    q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    s = np.ones(n, np.float32)
    c = _gemm(lib, bf16_dev(a), BF16, dev(q), I8, m, n, k, EPI_NONE, scales=dev(s))
    np.testing.assert_array_equal(host(c), a @ q.astype(np.float32).T)


@pytest.mark.parametrize("wdt", ["bf16", "i8"])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("m,n,k,epi", [(64, 512, 1024, EPI_NONE), (33, 256, 2048, EPI_RESIDUAL),
                                       (48, 128, 1536, EPI_SWIGLU), (64, 384, 4096, EPI_GLU_SILU_UP)])
def test_gemm_splitk_integer_operands(lib, wdt, layout, m, n, k, epi):
    """33..64 rows with a workspace run split-K over 512-k slices; on
    small-integer operands every partial sum is exact, so the result must equal
    the exact product and the single-pass kernel's (run with no workspace)."""
    assert lib.sfg_hip_gemm_workspace_v1(m, n, k) > 0
    rng = np.random.default_rng(m * 5 + n + k + layout)
    glu = epi in (EPI_SWIGLU, EPI_GLU_SILU_UP)
    nb = 2 * n if glu else n
    a = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
    res = rng.integers(-5, 6, size=(m, n)).astype(np.float32)
    if wdt == "bf16":
        b = rng.integers(-3, 4, size=(nb, k)).astype(np.float32)
        bd = dev(tile_nk(oracle.to_bf16_bits(b), "bf16").view(np.int16)) if layout else bf16_dev(b)
        bdt, sc = BF16, None
    else:
        q = rng.integers(-127, 128, size=(nb, k)).astype(np.int8)
        b = q.astype(np.float32)
        bd = dev(tile_nk(q, "int8")) if layout else dev(q)
        bdt, sc = I8, dev(np.ones(nb, np.float32))
    kw = dict(scales=sc, residual=dev(res) if epi == EPI_RESIDUAL else None, layout=layout)
    c = _gemm(lib, bf16_dev(a), BF16, bd, bdt, m, n, k, epi, **kw)
    c1 = _gemm(lib, bf16_dev(a), BF16, bd, bdt, m, n, k, epi, workspace=False, **kw)
    acc = a.astype(np.float64) @ b.T.astype(np.float64)
    ref = _ref_epilogue(acc, epi, n, res)
    if glu:
        np.testing.assert_allclose(host(c), ref, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(host(c), host(c1), rtol=1e-6, atol=1e-6)
    else:
        np.testing.assert_array_equal(host(c), ref.astype(np.float32))
        np.testing.assert_array_equal(host(c), host(c1))


@pytest.mark.parametrize("m,n,k,epi", [(128, 1376, 512, EPI_SWIGLU), (700, 688, 256, EPI_NONE),
                                       (300, 1376, 512, EPI_RESIDUAL), (1100, 1376, 256, EPI_SWIGLU),
                                       (1100, 688, 512, EPI_RESIDUAL)])
def test_gemm_bf16_ragged_n_integer_operands(lib, m, n, k, epi):
    """Output widths that are not a whole number of column tiles (the
    reference's tiny profile, intermediate 1376 = 10.75 x 128): the last tile's
    extra columns read a valid B row, are masked at the store, and every stored
    value is exact on small-integer operands."""
    rng = np.random.default_rng(m + 3 * n + k)
    glu = epi == EPI_SWIGLU
    a = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
    b = rng.integers(-3, 4, size=((2 * n) if glu else n, k)).astype(np.float32)
    res = rng.integers(-5, 6, size=(m, n)).astype(np.float32)
    c = _gemm(lib, bf16_dev(a), BF16, bf16_dev(b), BF16, m, n, k, epi,
              residual=dev(res) if epi == EPI_RESIDUAL else None)
    acc = a.astype(np.float64) @ b.T.astype(np.float64)
    ref = _ref_epilogue(acc, epi, n, res)
    if glu:
        np.testing.assert_allclose(host(c), ref, rtol=1e-5, atol=1e-5)
    else:
        np.testing.assert_array_equal(host(c), ref.astype(np.float32))


@pytest.mark.parametrize("m", [16, 64, 512, 1280])
@pytest.mark.parametrize("epi", [EPI_NONE, EPI_RESIDUAL, EPI_SWIGLU, EPI_GLU_SILU_UP])
def test_gemm_bf16_epilogues_match_oracle(lib, m, epi):
    n, k = 1024, 1024
    glu = epi in (EPI_SWIGLU, EPI_GLU_SILU_UP)
    a = oracle.round_bf16(oracle.normal(21, 0, (m, k)))
    b = oracle.round_bf16(oracle.normal(21, 2, (2 * n if glu else n, k), 0.02))
    res = oracle.normal(21, 5, (m, n))
    c = _gemm(lib, bf16_dev(a), BF16, bf16_dev(b), BF16, m, n, k, epi,
              residual=dev(res) if epi == EPI_RESIDUAL else None)
    acc = oracle.matmul(a, np.ascontiguousarray(b.T))
    ref = _ref_epilogue(acc, epi, n, res)
    assert oracle.rel_error(host(c), ref) < 1e-4


@pytest.mark.parametrize("m", [16, 64])
def test_gemm_int8_matches_oracle_quantized_matmul(lib, m):
    n, k = 2048, 1024
    w_kn = oracle.normal(31, 2, (k, n), 0.02)
    q, s = oracle.quantize_kn(w_kn)
    x = oracle.round_bf16(oracle.normal(31, 0, (m, k)))
    c = _gemm(lib, bf16_dev(x), BF16, dev(q), I8, m, n, k, EPI_NONE, scales=dev(s))
    ref = oracle.quantized_matmul(x, q, s)
    assert oracle.rel_error(host(c), ref) < 1e-4


@pytest.mark.parametrize("m,n,k,epi", [(128, 512, 256, EPI_NONE), (128, 256, 256, EPI_RESIDUAL),
                                       (128, 688, 256, EPI_SWIGLU), (128, 256, 688, EPI_RESIDUAL),
                                       (37, 100, 50, EPI_NONE)])
def test_gemm_f32_matches_oracle(lib, m, n, k, epi):
    glu = epi == EPI_SWIGLU
    a = oracle.normal(41, 0, (m, k))
    b = oracle.normal(41, 2, (2 * n if glu else n, k), 0.05)
    res = oracle.normal(41, 5, (m, n))
    c = _gemm(lib, dev(a), F32, dev(b), F32, m, n, k, epi,
              residual=dev(res) if epi == EPI_RESIDUAL else None)
    ref = _ref_epilogue(oracle.matmul(a, np.ascontiguousarray(b.T)), epi, n, res)
    assert oracle.rel_error(host(c), ref) < 1e-5


def test_gemm_rejects_bad_shapes(lib):
    args = _abi.GemmArgs()
    args.m = 0
    with pytest.raises(ValueError):
        _abi.check(lib.sfg_hip_gemm_v1(ctypes.byref(args), None, 0, stream()))


@pytest.mark.parametrize("wdt", ["bf16", "i8"])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("m,epi", [(20, EPI_NONE), (48, EPI_RESIDUAL), (64, EPI_NONE)])
def test_gemm_decode_gemv_widths_of_an_odd_number_of_16_column_tiles(lib, wdt, layout, m, epi):
    """17..64 decode rows take the decode GEMV on 32-column tiles; a width of
    624 = 39 x 16 columns runs it on 16-column tiles instead (with [N][K] and
    fragment-tiled weights alike), exact on small-integer operands."""
    n, k = 624, 2304
    rng = np.random.default_rng(m + layout)
    a = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
    res = rng.integers(-5, 6, size=(m, n)).astype(np.float32)
    if wdt == "bf16":
        b = rng.integers(-3, 4, size=(n, k)).astype(np.float32)
        bd = dev(tile_nk(oracle.to_bf16_bits(b), "bf16").view(np.int16)) if layout else bf16_dev(b)
        bdt, sc = BF16, None
    else:
        q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
        b = q.astype(np.float32)
        bd = dev(tile_nk(q, "int8")) if layout else dev(q)
        bdt, sc = I8, dev(np.ones(n, np.float32))
    c = _gemm(lib, bf16_dev(a), BF16, bd, bdt, m, n, k, epi, scales=sc, layout=layout,
              residual=dev(res) if epi == EPI_RESIDUAL else None, workspace=False)
    acc = a.astype(np.float64) @ b.T.astype(np.float64)
    np.testing.assert_array_equal(host(c), _ref_epilogue(acc, epi, n, res).astype(np.float32))


@pytest.mark.parametrize("tile", list(range(_abi.TILE_COUNT)))
@pytest.mark.parametrize("wdt,epi", [("bf16", EPI_NONE), ("bf16", EPI_SWIGLU), ("i8", EPI_GLU_SILU_UP)])
def test_gemm_grouped_gather_ids_outside_a_are_zero_rows(lib, tile, wdt, epi):
    """sfg_hip_gemm_grouped_v1 with a gather list holding ids outside
    [0, a_rows_limit) (-1 and past the end): those output rows are the
    product of a zero row (zero; the GLU epilogues of zeros are zero too),
    every other row the product of its gathered A row -- on the grouped
    MFMA kernels (3000 rows over five groups, one of them empty) under every
    tile policy.  Small-integer operands and power-of-two scales keep every
    value exact."""
    rng = np.random.default_rng(401 + tile)
    counts = [700, 0, 1100, 33, 1167]
    G, m, n, k, T = len(counts), sum(counts), 320, 256, 900
    glu = epi != EPI_NONE
    nb = 2 * n if glu else n
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    a = rng.integers(-3, 4, size=(T, k)).astype(np.float32)
    rows = rng.integers(0, T, size=m).astype(np.int32)
    rows[rng.random(m) < 0.05] = -1
    rows[rng.random(m) < 0.05] = T + 7
    rows[[0, 700, m - 1]] = [-1, T, T - 1]           # group edges
    if wdt == "i8":
        q = rng.integers(-127, 128, size=(G, nb, k)).astype(np.int8)
        s = rng.choice(np.array([0.5, 1.0, 2.0], np.float32), size=(G, nb)).astype(np.float32)
        bd, bdt, sd, s_stride = dev(q), I8, dev(s), nb
        bm = q.astype(np.float64) * s[..., None].astype(np.float64)
    else:
        b = rng.integers(-3, 4, size=(G, nb, k)).astype(np.float32)
        bd, bdt, sd, s_stride = bf16_dev(b), BF16, None, 0
        bm = b.astype(np.float64)
    ad, rd, od = bf16_dev(a), dev(rows), dev(offsets)
    c = torch.full((m, n), 7.0, dtype=torch.float32, device="cuda")   # stale contents
    args = _abi.GemmArgs()
    args.a, args.a_dtype, args.lda = ad.data_ptr(), BF16, k
    args.b, args.b_dtype, args.ldb = bd.data_ptr(), bdt, k
    args.b_scales = sd.data_ptr() if sd is not None else None
    args.c, args.c_dtype, args.ldc = c.data_ptr(), F32, n
    args.residual, args.ldr = None, n
    args.m, args.n, args.k, args.epilogue = m, n, k, epi
    args.b_layout, args.tile = 0, tile
    ws = torch.zeros(max(lib.sfg_hip_gemm_workspace_v1(m, n, k), 256), dtype=torch.uint8, device="cuda")
    _abi.check(lib.sfg_hip_gemm_grouped_v1(ctypes.byref(args), rd.data_ptr(), T, od.data_ptr(), G,
                                           nb * k, s_stride, ws.data_ptr(), ws.numel(), stream()))
    _sync()
    acc = np.zeros((m, nb))
    for g in range(G):
        src = rows[offsets[g]:offsets[g + 1]]
        valid = (src >= 0) & (src < T)
        arow = np.zeros((len(src), k))
        arow[valid] = a[src[valid]]
        acc[offsets[g]:offsets[g + 1]] = arow @ bm[g].T
    ref = _ref_epilogue(acc, epi, n)
    zero = (rows < 0) | (rows >= T)
    assert np.all(host(c)[zero] == 0.0)
    if glu:
        np.testing.assert_allclose(host(c), ref, rtol=1e-5, atol=1e-5)
    else:
        np.testing.assert_array_equal(host(c), ref.astype(np.float32))


def test_gemm_misaligned_operands_run_on_the_valu_kernel(lib):
    """bf16 / int8 MFMA kernels read rows as 16-byte vectors: a row pitch that
    is not a multiple of 16 bytes, or an operand not 16-byte aligned, runs on
    the VALU kernel instead (exact here: small integers)."""
    m, n, k = 16, 256, 256
    rng = np.random.default_rng(5)
    a32 = rng.integers(-2, 3, (m, k + 8)).astype(np.float32)
    b32 = rng.integers(-2, 3, (n, k)).astype(np.float32)
    a, b = bf16_dev(a32), bf16_dev(b32)
    c = torch.empty((m, n), dtype=torch.float32, device="cuda")
    flat = a32.reshape(-1)
    for lda, a_off in ((k + 1, 0), (k, 1)):  # odd pitch; base 2 bytes in
        args = _abi.GemmArgs()
        args.a, args.a_dtype, args.lda = a.data_ptr() + 2 * a_off, BF16, lda
        args.b, args.b_dtype, args.ldb, args.b_scales = b.data_ptr(), BF16, k, None
        args.c, args.c_dtype, args.ldc = c.data_ptr(), F32, n
        args.m, args.n, args.k, args.epilogue = m, n, k, EPI_NONE
        _abi.check(lib.sfg_hip_gemm_v1(ctypes.byref(args), None, 0, stream()))
        _sync()
        rows = np.stack([flat[a_off + r * lda: a_off + r * lda + k] for r in range(m)])
        np.testing.assert_array_equal(host(c), (rows.astype(np.float64) @ b32.T.astype(np.float64)))


# ------------------------------------------------------------------ packing
def test_pack_and_quantize_match_oracle(lib):
    k, n = 384, 640
    w = oracle.normal(51, 2, (k, n), 0.02)
    w[:, 3] = 0.0  # zero column -> scale 1
    wd = dev(w)
    dst = torch.empty((n, k), dtype=torch.int16, device="cuda")
    _abi.check(lib.sfg_hip_pack_weight_v1(wd.data_ptr(), k, n, n, dst.data_ptr(), BF16, 0, stream()))
    q = torch.empty((n, k), dtype=torch.int8, device="cuda")
    s = torch.empty((n,), dtype=torch.float32, device="cuda")
    _abi.check(lib.sfg_hip_quantize_weight_v1(wd.data_ptr(), k, n, q.data_ptr(), s.data_ptr(), 0, stream()))
    _sync()
    np.testing.assert_array_equal(host(dst).view(np.uint16), oracle.to_bf16_bits(w.T))
    qr, sr = oracle.quantize_kn(w)
    np.testing.assert_array_equal(host(q), qr)
    np.testing.assert_array_equal(host(s), sr)
    assert host(s)[3] == 1.0


# ------------------------------------------------------------------ split + RoPE
@pytest.mark.parametrize("dtype", [F32, BF16])
def test_split_rope_matches_oracle(lib, dtype):
    B, S, Hq, Hkv, D, theta = 2, 40, 4, 2, 64, 10000.0
    H = Hq * D
    qkv = oracle.normal(61, 0, (B * S, H + 2 * Hkv * D))
    table = np.empty((S, D // 2, 2), np.float32)
    _abi.check(lib.sfg_hip_rope_table_host_v1(table.ctypes.data, S, D, ctypes.c_float(theta)))
    tdt = torch.float32 if dtype == F32 else torch.int16
    q = torch.empty((B, Hq, S, D), dtype=tdt, device="cuda")
    k = torch.empty((B, Hkv, S, D), dtype=tdt, device="cuda")
    v = torch.empty((B, Hkv, S, D), dtype=tdt, device="cuda")
    _abi.check(lib.sfg_hip_qkv_split_rope_v1(dev(qkv).data_ptr(), dev(table).data_ptr(), B, S, Hq,
                                             Hkv, D, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                             dtype, stream()))
    _sync()
    rq, rk, rv = oracle.split_qkv_rope(qkv, B, S, H, Hq, Hkv, D, theta)
    conv = host if dtype == F32 else bf16_host
    tol = 1e-6 if dtype == F32 else 8e-3
    for got, ref in ((q, rq), (k, rk), (v, rv)):
        assert oracle.rel_error(conv(got), ref) < tol
    # position 0 is the identity rotation
    exact_v = rv if dtype == F32 else oracle.round_bf16(rv)
    np.testing.assert_array_equal(conv(v)[:, :, 0], exact_v[:, :, 0])


@pytest.mark.parametrize("dtype", [F32, BF16])
@pytest.mark.parametrize("D", [1, 5, 33])
def test_split_rope_odd_head_dims(lib, dtype, D):
    """An odd head_dim's last dimension is copied unrotated, as apply_rope's
    pair loop (decoder_compiler.cpp:101-114, d + 1 < D) leaves it; head_dim 1
    has no pair and needs no table."""
    B, S, Hq, Hkv, theta = 2, 23, 6, 2, 10000.0
    H = Hq * D
    qkv = oracle.normal(62, D, (B * S, H + 2 * Hkv * D))
    table = np.zeros((S, max(D // 2, 1), 2), np.float32)
    _abi.check(lib.sfg_hip_rope_table_host_v1(table.ctypes.data, S, D, ctypes.c_float(theta)))
    tdt = torch.float32 if dtype == F32 else torch.int16
    q = torch.empty((B, Hq, S, D), dtype=tdt, device="cuda")
    k = torch.empty((B, Hkv, S, D), dtype=tdt, device="cuda")
    v = torch.empty((B, Hkv, S, D), dtype=tdt, device="cuda")
    _abi.check(lib.sfg_hip_qkv_split_rope_v1(dev(qkv).data_ptr(), dev(table).data_ptr() if D > 1 else None,
                                             B, S, Hq, Hkv, D, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                             dtype, stream()))
    _sync()
    rq, rk, rv = oracle.split_qkv_rope(qkv, B, S, H, Hq, Hkv, D, theta)
    conv = host if dtype == F32 else bf16_host
    exact = (lambda a: a) if dtype == F32 else oracle.round_bf16
    for got, ref in ((q, rq), (k, rk), (v, rv)):
        assert oracle.rel_error(conv(got), ref) < (1e-6 if dtype == F32 else 8e-3)
        # the last (unpaired) dimension is the input's, exactly
        np.testing.assert_array_equal(conv(got)[..., D - 1], exact(ref)[..., D - 1])


# ------------------------------------------------------------------ attention
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(1, 4, 2, 128, 128, 64), (2, 4, 1, 33, 70, 64),
                                   (1, 2, 2, 5, 5, 16)])
def test_attention_prefill_f32_matches_oracle(lib, causal, shape):
    B, Hq, Hkv, Sq, Skv, D = shape
    if causal and Sq > Skv:
        pytest.skip("invalid")
    q = oracle.normal(71, 0, (B, Hq, Sq, D))
    k = oracle.normal(71, 1, (B, Hkv, Skv, D))
    v = oracle.normal(71, 2, (B, Hkv, Skv, D))
    out = torch.empty((B * Sq, Hq * D), dtype=torch.float32, device="cuda")
    _abi.check(lib.sfg_hip_attn_prefill_v1(dev(q).data_ptr(), dev(k).data_ptr(), dev(v).data_ptr(),
                                           out.data_ptr(), F32, F32, B, Hq, Hkv, Sq, Skv, D,
                                           int(causal), ctypes.c_float(0.0), stream()))
    _sync()
    ref = oracle.attention(q, k, v, causal).transpose(0, 2, 1, 3).reshape(B * Sq, Hq * D)
    assert oracle.rel_error(host(out), ref) < 1e-5


@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(1, 4, 2, 256, 256), (2, 8, 2, 300, 300), (1, 2, 1, 64, 200),
                                   (1, 2, 2, 1, 77)])
def test_attention_prefill_bf16_matches_oracle(lib, causal, shape, D):
    B, Hq, Hkv, Sq, Skv = shape
    q = oracle.round_bf16(oracle.normal(81, 0, (B, Hq, Sq, D)))
    k = oracle.round_bf16(oracle.normal(81, 1, (B, Hkv, Skv, D)))
    v = oracle.round_bf16(oracle.normal(81, 2, (B, Hkv, Skv, D)))
    out = torch.empty((B * Sq, Hq * D), dtype=torch.float32, device="cuda")
    _abi.check(lib.sfg_hip_attn_prefill_v1(bf16_dev(q).data_ptr(), bf16_dev(k).data_ptr(),
                                           bf16_dev(v).data_ptr(), out.data_ptr(), BF16, F32, B,
                                           Hq, Hkv, Sq, Skv, D, int(causal), ctypes.c_float(0.0),
                                           stream()))
    _sync()
    ref = oracle.attention(q, k, v, causal).transpose(0, 2, 1, 3).reshape(B * Sq, Hq * D)
    assert oracle.rel_error(host(out), ref) < 2e-2


def test_attention_prefill_bf16_equal_keys_is_prefix_mean(lib):
    """Equal keys: causal softmax is uniform over the prefix, so row i of the
    output is the mean of V[0..i] (a closed form independent of the oracle)."""
    B, Hq, Hkv, S, D = 1, 2, 1, 192, 128
    q = oracle.round_bf16(oracle.normal(82, 0, (B, Hq, S, D)))
    krow = oracle.round_bf16(oracle.normal(82, 1, (D,)))
    k = np.broadcast_to(krow, (B, Hkv, S, D)).copy()
    v = oracle.round_bf16(oracle.normal(82, 2, (B, Hkv, S, D)))
    out = torch.empty((B * S, Hq * D), dtype=torch.float32, device="cuda")
    _abi.check(lib.sfg_hip_attn_prefill_v1(bf16_dev(q).data_ptr(), bf16_dev(k).data_ptr(),
                                           bf16_dev(v).data_ptr(), out.data_ptr(), BF16, F32, B,
                                           Hq, Hkv, S, S, D, 1, ctypes.c_float(0.0), stream()))
    _sync()
    prefix = np.cumsum(v[0, 0].astype(np.float64), axis=0) / np.arange(1, S + 1)[:, None]
    got = host(out).reshape(S, Hq, D)
    for h in range(Hq):
        assert np.max(np.abs(got[:, h] - prefix)) < 2e-2


# ------------------------------------------------------- flash prefill over V^T
def _vt_host(v, ld):
    """[B][Hkv][S][D] -> [B][Hkv][D][ld] with keys >= S zero."""
    B, Hkv, S, D = v.shape
    vt = np.zeros((B, Hkv, D, ld), np.float32)
    vt[..., :S] = v.transpose(0, 1, 3, 2)
    return vt


def _prefill_vt(lib, q, k, v, causal, out_dtype=F32):
    B, Hq, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    ld = lib.sfg_hip_attn_vt_ld_v1(Skv)
    assert ld % 64 == 0 and ld >= Skv
    tdt = torch.float32 if out_dtype == F32 else torch.int16
    out = torch.empty((B * Sq, Hq * D), dtype=tdt, device="cuda")
    _abi.check(lib.sfg_hip_attn_prefill_vt_v1(bf16_dev(q).data_ptr(), bf16_dev(k).data_ptr(),
                                              bf16_dev(_vt_host(v, ld)).data_ptr(), ld,
                                              out.data_ptr(), out_dtype, B, Hq, Hkv, Sq, Skv, D,
                                              int(causal), ctypes.c_float(0.0), stream()))
    _sync()
    return host(out) if out_dtype == F32 else bf16_host(out)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(1, 4, 2, 256, 256), (2, 8, 2, 300, 300), (1, 2, 1, 64, 200),
                                   (1, 2, 2, 1, 77), (1, 8, 1, 1000, 1000), (2, 4, 4, 130, 190),
                                   (1, 16, 2, 520, 520)])
def test_attention_prefill_vt_matches_oracle(lib, causal, shape):
    B, Hq, Hkv, Sq, Skv = shape
    D = 128
    q = oracle.round_bf16(oracle.normal(83, 0, (B, Hq, Sq, D)))
    k = oracle.round_bf16(oracle.normal(83, 1, (B, Hkv, Skv, D)))
    v = oracle.round_bf16(oracle.normal(83, 2, (B, Hkv, Skv, D)))
    got = _prefill_vt(lib, q, k, v, causal)
    ref = oracle.attention(q, k, v, causal).transpose(0, 2, 1, 3).reshape(B * Sq, Hq * D)
    assert np.isfinite(got).all()
    assert oracle.rel_error(got, ref) < 2e-2


def test_attention_prefill_vt_large_scores_stay_exact(lib):
    """Scores spanning a wide range (scaled Q) exercise the lazy rescale: a
    row's max moves by far more than the 2^8 slack several times."""
    B, Hq, Hkv, S, D = 1, 2, 1, 384, 128
    ramp = np.linspace(0.2, 6.0, S, dtype=np.float32)[None, None, :, None]
    q = oracle.round_bf16(oracle.normal(84, 0, (B, Hq, S, D)) * 3.0)
    k = oracle.round_bf16(oracle.normal(84, 1, (B, Hkv, S, D)) * ramp)
    v = oracle.round_bf16(oracle.normal(84, 2, (B, Hkv, S, D)))
    for causal in (True, False):
        got = _prefill_vt(lib, q, k, v, causal)
        ref = oracle.attention(q, k, v, causal).transpose(0, 2, 1, 3).reshape(B * S, Hq * D)
        assert oracle.rel_error(got, ref) < 2e-2


def test_attention_prefill_vt_equal_keys_is_prefix_mean(lib):
    """Closed form: equal keys make causal softmax uniform over the prefix."""
    B, Hq, Hkv, S, D = 1, 2, 1, 200, 128
    q = oracle.round_bf16(oracle.normal(85, 0, (B, Hq, S, D)))
    k = np.broadcast_to(oracle.round_bf16(oracle.normal(85, 1, (D,))), (B, Hkv, S, D)).copy()
    v = oracle.round_bf16(oracle.normal(85, 2, (B, Hkv, S, D)))
    got = _prefill_vt(lib, q, k, v, True, out_dtype=BF16).reshape(S, Hq, D)
    prefix = np.cumsum(v[0, 0].astype(np.float64), axis=0) / np.arange(1, S + 1)[:, None]
    for h in range(Hq):
        assert np.max(np.abs(got[:, h] - prefix)) < 2e-2


def test_attention_prefill_vt_s8192_matches_oracle_rows(lib):
    """C4's sequence length (8192) with few heads: the flash kernel over the
    whole causal range, checked on the first, a middle and the last 256 query
    rows.  Causal alignment (j <= Skv - Sq + i, attention_compiler.cpp:68-72)
    lets the oracle run a row block against exactly the key prefix it sees."""
    B, Hq, Hkv, S, D = 1, 4, 1, 8192, 128
    q = oracle.round_bf16(oracle.normal(86, 0, (B, Hq, S, D)))
    k = oracle.round_bf16(oracle.normal(86, 1, (B, Hkv, S, D)))
    v = oracle.round_bf16(oracle.normal(86, 2, (B, Hkv, S, D)))
    got = _prefill_vt(lib, q, k, v, True).reshape(S, Hq, D)
    assert np.isfinite(got).all()
    for r0 in (0, 4000, S - 256):
        r1 = r0 + 256
        ref = oracle.attention(q[:, :, r0:r1], k[:, :, :r1], v[:, :, :r1], True)[0].transpose(1, 0, 2)
        err = oracle.rel_error(got[r0:r1], ref)
        print(f"S8192 rows [{r0}, {r1}): rel_err {err:.3e}")
        assert err < 2e-2


def test_attention_prefill_vt_s8192_equal_keys_is_prefix_mean(lib):
    """Closed form at S 8192: equal keys give every allowed key probability
    exactly 1 before normalisation, so row i is the mean of V[0..i]."""
    B, Hq, Hkv, S, D = 1, 2, 1, 8192, 128
    q = oracle.round_bf16(oracle.normal(87, 0, (B, Hq, S, D)))
    k = np.broadcast_to(oracle.round_bf16(oracle.normal(87, 1, (D,))), (B, Hkv, S, D)).copy()
    v = oracle.round_bf16(oracle.normal(87, 2, (B, Hkv, S, D)))
    got = _prefill_vt(lib, q, k, v, True).reshape(S, Hq, D)
    prefix = np.cumsum(v[0, 0].astype(np.float64), axis=0) / np.arange(1, S + 1)[:, None]
    for h in range(Hq):
        err = np.max(np.abs(got[:, h] - prefix))
        print(f"S8192 equal keys head {h}: max abs err {err:.2e}")
        assert err < 1e-3


def test_split_rope_vt_matches_split_rope(lib):
    """split_qkv + RoPE writing V^T: q and k bit-equal to the plain split, vt
    the exact transpose of its v with zero key padding."""
    B, S, Hq, Hkv, D = 2, 100, 4, 2, 128
    H = Hq * D
    qkv = oracle.normal(62, 0, (B * S, H + 2 * Hkv * D))
    table = np.empty((S, D // 2, 2), np.float32)
    _abi.check(lib.sfg_hip_rope_table_host_v1(table.ctypes.data, S, D, ctypes.c_float(1e4)))
    qkv_d, table_d = dev(qkv), dev(table)
    q, k, v = (torch.empty((B, h, S, D), dtype=torch.int16, device="cuda") for h in (Hq, Hkv, Hkv))
    _abi.check(lib.sfg_hip_qkv_split_rope_v1(qkv_d.data_ptr(), table_d.data_ptr(), B, S, Hq, Hkv,
                                             D, q.data_ptr(), k.data_ptr(), v.data_ptr(), BF16,
                                             stream()))
    ld = lib.sfg_hip_attn_vt_ld_v1(S)
    q2 = torch.empty_like(q)
    k2 = torch.empty_like(k)
    vt = torch.full((B, Hkv, D, ld), 0x7FC0, dtype=torch.int16, device="cuda")  # NaN fill
    _abi.check(lib.sfg_hip_qkv_split_rope_vt_v1(qkv_d.data_ptr(), table_d.data_ptr(), B, S, Hq,
                                                Hkv, D, q2.data_ptr(), k2.data_ptr(), vt.data_ptr(),
                                                ld, stream()))
    _sync()
    np.testing.assert_array_equal(host(q2), host(q))
    np.testing.assert_array_equal(host(k2), host(k))
    expect = np.zeros((B, Hkv, D, ld), np.int16)
    expect[..., :S] = host(v).transpose(0, 1, 3, 2)
    np.testing.assert_array_equal(host(vt), expect)
    with pytest.raises(ValueError):
        _abi.check(lib.sfg_hip_qkv_split_rope_vt_v1(qkv_d.data_ptr(), table_d.data_ptr(), B, S,
                                                    Hq, Hkv, D, q2.data_ptr(), k2.data_ptr(),
                                                    vt.data_ptr(), ld + 1, stream()))


def _decode_case(lib, B, Hq, Hkv, ctx, seq_lens=None, splits=0, seed=91, D=128):
    PT = 16
    pps = (ctx + PT - 1) // PT
    num_pages = B * pps + 3
    perm = oracle.page_permutation(seed, num_pages)[: B * pps]
    table = perm.reshape(B, pps).astype(np.int32)
    kc = oracle.round_bf16(oracle.normal(seed, 15, (B, Hkv, ctx, D)))
    vc = oracle.round_bf16(oracle.normal(seed, 16, (B, Hkv, ctx, D)))
    q = oracle.normal(seed, 0, (B, Hq, 1, D))
    kp = oracle.paged_scatter(kc, table, num_pages, PT)
    vp = oracle.paged_scatter(vc, table, num_pages, PT)
    vp_t = np.ascontiguousarray(vp.transpose(0, 1, 3, 2))  # V pool is token-minor per page
    out = torch.empty((B, Hq * D), dtype=torch.float32, device="cuda")
    wsb = lib.sfg_hip_attn_decode_workspace_v1(B, Hq, D, ctx, PT, splits)
    ws = torch.zeros(wsb, dtype=torch.uint8, device="cuda")
    sl = dev(np.asarray(seq_lens, np.int32)) if seq_lens is not None else None
    _abi.check(lib.sfg_hip_attn_decode_paged_v1(
        dev(q).data_ptr(), bf16_dev(kp).data_ptr(), bf16_dev(vp_t).data_ptr(), dev(table).data_ptr(),
        sl.data_ptr() if sl is not None else None, out.data_ptr(), F32, B, Hq, Hkv, D, PT, pps,
        num_pages, ctx, splits, ctypes.c_float(0.0), 1, ws.data_ptr(), ws.numel(), stream()))
    _sync()
    got = host(out).reshape(B, Hq, D)
    for b in range(B):
        L = ctx if seq_lens is None else seq_lens[b]
        # gather through the table, then the reference attention (decode: Sq=1 sees all keys)
        flat_k = oracle.paged_gather(kp, table[b:b + 1], 1, Hkv, L, PT, D)
        flat_v = oracle.paged_gather(vp, table[b:b + 1], 1, Hkv, L, PT, D)
        ref = oracle.attention(q[b:b + 1], flat_k, flat_v, True)[0, :, 0]
        assert oracle.rel_error(got[b], ref) < 2e-2, b
    return got


@pytest.mark.parametrize("B,Hq,Hkv,ctx", [(4, 8, 2, 1000), (2, 16, 4, 4096), (3, 4, 4, 17),
                                          (2, 8, 1, 256), (1, 32, 4, 50)])
def test_decode_paged_matches_oracle(lib, B, Hq, Hkv, ctx):
    _decode_case(lib, B, Hq, Hkv, ctx)


@pytest.mark.parametrize("B,Hq,Hkv,ctx", [(1, 8, 2, 512), (3, 16, 4, 100), (2, 4, 4, 2048)])
def test_decode_paged_head_dim_64_matches_oracle(lib, B, Hq, Hkv, ctx):
    """head_dim 64 (the reference's tiny / medium decoder profiles,
    decoder_compiler.cpp:920-921): two S^T k-steps and four O^T blocks per page."""
    _decode_case(lib, B, Hq, Hkv, ctx, D=64)
    _decode_case(lib, B, Hq, Hkv, ctx, D=64, splits=3, seed=92)


@pytest.mark.parametrize("ctx,lens", [(4096, None), (6000, None), (6000, [6000, 1500, 17, 4097])])
def test_decode_long_page_ranges_match_oracle(lib, ctx, lens):
    """One split: each wave walks more than 16 pages (64 and about 94), so the
    page ids come 64 at a time from one vector load, reloaded past 64 pages."""
    B = 4 if lens else 2
    _decode_case(lib, B, 8, 2, ctx, seq_lens=np.array(lens, np.int32) if lens else None, splits=1, seed=93)


def test_decode_ragged_lengths_and_split_invariance(lib):
    lens = [1000, 1, 513, 640]
    a = _decode_case(lib, 4, 8, 2, 1000, seq_lens=lens, splits=1)
    b = _decode_case(lib, 4, 8, 2, 1000, seq_lens=lens, splits=8)
    # merge_online is exact up to rounding: any split count gives the same
    # result; P enters the value MFMA as bf16 after a split-dependent max
    # shift, so the two agree to bf16 rounding.
    assert oracle.rel_error(a, b) < 1e-2


def test_decode_rejects_bad_page_ids(lib):
    B, Hq, Hkv, D, PT, ctx = 1, 4, 1, 128, 16, 32
    table = np.array([[0, 99]], np.int32)
    pool = torch.zeros((2, Hkv, PT, D), dtype=torch.int16, device="cuda")
    q = torch.zeros((B, Hq, D), dtype=torch.float32, device="cuda")
    out = torch.empty((B, Hq * D), dtype=torch.float32, device="cuda")
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError, match="invalid physical KV page"):
        _abi.check(lib.sfg_hip_attn_decode_paged_v1(
            q.data_ptr(), pool.data_ptr(), pool.data_ptr(), dev(table).data_ptr(), None,
            out.data_ptr(), F32, B, Hq, Hkv, D, PT, 2, 2, ctx, 0, ctypes.c_float(0.0), 1,
            ws.data_ptr(), ws.numel(), stream()))
    with pytest.raises(ValueError, match="compiled guard"):
        _abi.check(lib.sfg_hip_attn_decode_paged_v1(
            q.data_ptr(), pool.data_ptr(), pool.data_ptr(), dev(table).data_ptr(), None,
            out.data_ptr(), F32, B, Hq, Hkv, D, PT, 2, 2, 33, 0, ctypes.c_float(0.0), 0,
            ws.data_ptr(), ws.numel(), stream()))


# ------------------------------------------------------------------ MoE routing
def _route(lib, x, router, bias, top_k):
    T, H = x.shape
    E = router.shape[1]
    ids = torch.empty((T, top_k), dtype=torch.int32, device="cuda")
    w = torch.empty((T, top_k), dtype=torch.float32, device="cuda")
    counts = torch.empty(E, dtype=torch.int32, device="cuda")
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    tok = torch.empty(T * top_k, dtype=torch.int32, device="cuda")
    slots = torch.empty(T * top_k, dtype=torch.int32, device="cuda")
    rw = torch.empty(T * top_k, dtype=torch.float32, device="cuda")
    pos = torch.empty(T * top_k, dtype=torch.int32, device="cuda")
    bd = dev(bias) if bias is not None else None
    _abi.check(lib.sfg_hip_moe_route_v1(dev(x).data_ptr(), dev(router).data_ptr(),
                                        bd.data_ptr() if bd is not None else None, T, H, E, top_k,
                                        ids.data_ptr(), w.data_ptr(), counts.data_ptr(),
                                        offsets.data_ptr(), tok.data_ptr(), slots.data_ptr(),
                                        rw.data_ptr(), pos.data_ptr(), None, 0, stream()))
    _sync()
    return [host(t) for t in (ids, w, counts, offsets, tok, slots, rw, pos)]


@pytest.mark.parametrize("T,H,E,k,bias_std", [(2048, 2048, 8, 2, 0.5), (64, 4096, 8, 2, 0.0),
                                              (100, 512, 16, 4, 1.0), (33, 256, 4, 1, 0.0),
                                              # six 512-feature router chunks, ragged last workgroup
                                              (37, 3072, 8, 2, 0.5),
                                              # dispatch held in registers: 8 full chunks of
                                              # 1024 assignments; a ragged last chunk
                                              (4096, 128, 16, 2, 1.0), (1537, 256, 8, 2, 0.5),
                                              # chunked dispatch: more experts / assignments
                                              (300, 256, 32, 2, 1.0), (5000, 128, 8, 2, 0.5),
                                              # the reference's MoE test shape (test_schedforge.cpp:617)
                                              (7, 8, 4, 2, 0.0)])
def test_moe_route_bit_exact(lib, T, H, E, k, bias_std):
    x = oracle.normal(101, 0, (T, H))
    router = oracle.normal(101, 10, (H, E), 0.02)
    bias = oracle.normal(101, 11, (E,), bias_std) if bias_std > 0 else None
    ids, w, counts, offsets, tok, slots, rw, pos = _route(lib, x, router, bias, k)
    rids, rwts, rcounts = oracle.route_topk(x, router, bias, k)
    np.testing.assert_array_equal(ids, rids)
    np.testing.assert_allclose(w, rwts, rtol=2e-6, atol=0)
    np.testing.assert_array_equal(counts, rcounts)
    c2, roff, rtok, rslots, rrw = oracle.dispatch(rids, rwts, E)
    np.testing.assert_array_equal(offsets, roff)
    np.testing.assert_array_equal(tok, rtok)
    np.testing.assert_array_equal(slots, rslots)
    # position is the inverse permutation of (token, slot) -> dispatched row
    np.testing.assert_array_equal(tok[pos], np.repeat(np.arange(T), k))
    np.testing.assert_array_equal(slots[pos], np.tile(np.arange(k), T))
    np.testing.assert_allclose(rw, rrw, rtol=2e-6)


def test_moe_route_ties_go_to_lower_expert(lib):
    """Identical router columns give exactly equal logits: the lower expert
    index must win every tie."""
    T, H, E = 256, 512, 8
    x = oracle.normal(102, 0, (T, H))
    router = oracle.normal(102, 10, (H, E), 0.02)
    router[:, 5] = router[:, 2]
    router[:, 7] = router[:, 2]
    ids, *_ = _route(lib, x, router, None, 2)
    rids, _, _ = oracle.route_topk(x, router, None, 2)
    np.testing.assert_array_equal(ids, rids)
    for t in range(T):
        chosen = set(ids[t].tolist())
        if 5 in chosen:
            assert 2 in chosen
        if 7 in chosen:
            assert 2 in chosen and 5 in chosen


@pytest.mark.parametrize("T,E", [(300, 8), (300, 32)])   # register and chunked dispatch
def test_moe_dispatch_trace_skips_out_of_range_experts(lib, T, E):
    """A caller-supplied routing trace with expert ids outside [0, E) (the
    reference refuses them, next_milestones.cpp:427-428): such an assignment is
    left out of the histogram and the segments, its position is -1, and the
    combine adds nothing for it (the token keeps its other slots)."""
    k, H = 2, 256
    rng = np.random.default_rng(7)
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    ids[5, 0], ids[77, 1], ids[299, 0] = E, -1, E + 100
    w = rng.random((T, k)).astype(np.float32)
    counts = torch.empty(E, dtype=torch.int32, device="cuda")
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    tok = torch.full((T * k,), -7, dtype=torch.int32, device="cuda")
    slots = torch.empty(T * k, dtype=torch.int32, device="cuda")
    rw = torch.empty(T * k, dtype=torch.float32, device="cuda")
    pos = torch.full((T * k,), 12345, dtype=torch.int32, device="cuda")  # stale contents
    _abi.check(lib.sfg_hip_moe_dispatch_trace_v1(dev(ids).data_ptr(), dev(w).data_ptr(), T, E, k,
                                                 counts.data_ptr(), offsets.data_ptr(),
                                                 tok.data_ptr(), slots.data_ptr(), rw.data_ptr(),
                                                 pos.data_ptr(), stream()))
    _sync()
    valid = (ids >= 0) & (ids < E)
    np.testing.assert_array_equal(host(counts), np.bincount(ids[valid], minlength=E))
    p = host(pos).reshape(T, k)
    assert p[5, 0] == -1 and p[77, 1] == -1 and p[299, 0] == -1
    n_valid = int(valid.sum())
    assert host(offsets)[E] == n_valid
    np.testing.assert_array_equal(np.sort(p[valid]), np.arange(n_valid))
    y = oracle.normal(112, 0, (T * k, H))
    resid = oracle.normal(112, 5, (T, H))
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    _abi.check(lib.sfg_hip_moe_combine_v1(dev(y).data_ptr(), pos.data_ptr(), dev(w).data_ptr(),
                                          dev(resid).data_ptr(), out.data_ptr(), T, H, k, stream()))
    _sync()
    ref = resid.copy()
    for t in range(T):
        for s in range(k):
            if valid[t, s]:
                ref[t] = np.float32(ref[t] + w[t, s] * y[p[t, s]])
    assert oracle.rel_error(host(out), ref) < 1e-6
    np.testing.assert_allclose(host(out)[5] - resid[5], w[5, 1] * y[p[5, 1]], rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ MoE experts + combine
@pytest.mark.parametrize("wdt", ["bf16", "w8"])
@pytest.mark.parametrize("T,layout,H,I,E", [(256, 0, 512, 256, 8), (16, 0, 512, 256, 8),
                                             (700, 0, 512, 256, 8), (1500, 0, 512, 256, 8),
                                             (16, 1, 512, 256, 8), (256, 1, 512, 256, 8),
                                             # the reference's MoE test shape, MoeConfig{7, 8, 12, 4, 2}
                                             # (test_schedforge.cpp:617): k of 8 and 12 take the VALU kernel
                                             (7, 0, 8, 12, 4)])
def test_moe_experts_and_combine_match_oracle(lib, wdt, T, layout, H, I, E):
    """Grouped expert GEMMs + combine; layout 1 = fragment-tiled weights (decode sizes only)."""
    k = 2
    x = oracle.round_bf16(oracle.normal(111, 0, (T, H)))
    router = oracle.normal(111, 10, (H, E), 0.02)
    bias = oracle.normal(111, 11, (E,), 1.0)
    ids, w, counts, offsets, tok, slots, rw, pos = _route(lib, x, router, bias, k)
    _check_experts_and_combine(lib, wdt, layout, x, ids, w, offsets, tok, pos, H, I, E, k)


def _dispatch_trace(lib, ids, w, E):
    T, k = ids.shape
    counts = torch.empty(E, dtype=torch.int32, device="cuda")
    offsets = torch.empty(E + 1, dtype=torch.int32, device="cuda")
    tok = torch.empty(T * k, dtype=torch.int32, device="cuda")
    slots = torch.empty(T * k, dtype=torch.int32, device="cuda")
    rw = torch.empty(T * k, dtype=torch.float32, device="cuda")
    pos = torch.empty(T * k, dtype=torch.int32, device="cuda")
    _abi.check(lib.sfg_hip_moe_dispatch_trace_v1(dev(ids).data_ptr(), dev(w).data_ptr(), T, E, k,
                                                 counts.data_ptr(), offsets.data_ptr(),
                                                 tok.data_ptr(), slots.data_ptr(), rw.data_ptr(),
                                                 pos.data_ptr(), stream()))
    _sync()
    return host(counts), host(offsets), host(tok), host(pos)


@pytest.mark.parametrize("wdt", ["bf16", "w8"])
@pytest.mark.parametrize("T,layout", [(16, 1), (256, 1), (256, 0), (1500, 0)])
def test_moe_experts_with_every_token_on_two_experts(lib, wdt, T, layout):
    """The most skewed routing a top-2 trace can give: every token on experts
    0 and E - 1, the six experts between them empty.  One group then holds T
    rows -- 16 and 256 rows take the grouped decode GEMV (256 x 2 = 512
    assignments is its largest grouped problem, 16 passes of 32 rows over one
    expert), 1500 rows the grouped MFMA tiles -- while the empty groups launch
    workgroups that must store nothing."""
    H, I, E, k = 512, 256, 8, 2
    x = oracle.round_bf16(oracle.normal(113, 0, (T, H)))
    rng = np.random.default_rng(113)
    ids = np.where(rng.random((T, 1)) < 0.5, [[0, E - 1]], [[E - 1, 0]]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    counts, offsets, tok, pos = _dispatch_trace(lib, ids, w, E)
    assert counts[0] == T and counts[E - 1] == T and counts[1:E - 1].sum() == 0
    _check_experts_and_combine(lib, wdt, layout, x, ids, w, offsets, tok, pos, H, I, E, k, seed=113)


def _check_experts_and_combine(lib, wdt, layout, x, ids, w, offsets, tok, pos, H, I, E, k, seed=111):
    """Grouped expert GEMMs (sfg_hip_moe_experts_v1) and the weighted combine
    for a routing (ids, w) already dispatched, against the oracle's MoE."""
    T = x.shape[0]
    w1 = oracle.normal(seed, 12, (E, H, I), 0.02)
    w3 = oracle.normal(seed, 13, (E, H, I), 0.02)
    w2 = oracle.normal(seed, 14, (E, I, H), 0.02)
    if wdt == "bf16":
        w1, w3, w2 = (oracle.round_bf16(m) for m in (w1, w3, w2))
    # device weights in [E][2I][H] / [E][H][I]
    if wdt == "bf16":
        w13 = np.concatenate([w1.transpose(0, 2, 1), w3.transpose(0, 2, 1)], axis=1)
        w2t = np.ascontiguousarray(w2.transpose(0, 2, 1))
        if layout:
            w13d = dev(np.stack([tile_nk(oracle.to_bf16_bits(w13[e]), "bf16") for e in range(E)]).view(np.int16))
            w2d = dev(np.stack([tile_nk(oracle.to_bf16_bits(w2t[e]), "bf16") for e in range(E)]).view(np.int16))
        else:
            w13d, w2d = bf16_dev(np.ascontiguousarray(w13)), bf16_dev(w2t)
        s13d = s2d = None
        dt = BF16
    else:
        q1 = [oracle.quantize_kn(w1[e]) for e in range(E)]
        q3 = [oracle.quantize_kn(w3[e]) for e in range(E)]
        q2 = [oracle.quantize_kn(w2[e]) for e in range(E)]
        q13 = [np.concatenate([q1[e][0], q3[e][0]]) for e in range(E)]
        w13d = dev(np.stack([tile_nk(q, "int8") if layout else q for q in q13]))
        s13d = dev(np.stack([np.concatenate([q1[e][1], q3[e][1]]) for e in range(E)]))
        w2d = dev(np.stack([tile_nk(q2[e][0], "int8") if layout else q2[e][0] for e in range(E)]))
        s2d = dev(np.stack([q2[e][1] for e in range(E)]))
        dt = I8
    act = torch.empty((T * k, I), dtype=torch.int16, device="cuda")
    y = torch.empty((T * k, H), dtype=torch.float32, device="cuda")
    _abi.check(lib.sfg_hip_moe_experts_v1(bf16_dev(x).data_ptr(), dev(offsets).data_ptr(),
                                          dev(tok).data_ptr(), w13d.data_ptr(),
                                          s13d.data_ptr() if s13d is not None else None,
                                          w2d.data_ptr(), s2d.data_ptr() if s2d is not None else None,
                                          dt, layout, act.data_ptr(), y.data_ptr(), T, H, I, E, k, None, 0,
                                          stream()))
    resid = oracle.normal(seed, 5, (T, H))
    out = torch.empty((T, H), dtype=torch.float32, device="cuda")
    _abi.check(lib.sfg_hip_moe_combine_v1(y.data_ptr(), dev(pos).data_ptr(), dev(w).data_ptr(),
                                          dev(resid).data_ptr(), out.data_ptr(), T, H, k, stream()))
    _sync()
    if wdt == "bf16":
        ffn = oracle.moe_reference(x, w1, w3, w2, ids, w)
    else:
        from oracle import _b, _f, _i, i64, lib as olib
        ffn = np.empty((T, H), np.float32)
        e1q, e1s = np.stack([q[0] for q in q1]), np.stack([q[1] for q in q1])
        e3q, e3s = np.stack([q[0] for q in q3]), np.stack([q[1] for q in q3])
        e2q, e2s = np.stack([q[0] for q in q2]), np.stack([q[1] for q in q2])
        olib().sfgo_quantized_moe(_f(x), _b(e1q), _f(e1s), _b(e3q), _f(e3s), _b(e2q), _f(e2s),
                                  i64(T), i64(H), i64(I), i64(k), _i(ids), _f(w), _f(ffn))
    ref = resid + ffn
    tol = 2e-2 if wdt == "bf16" else 1e-2
    assert oracle.rel_error(host(out), ref) < tol
    # FFN part alone (residual removed) within the same tolerance
    assert oracle.rel_error(host(out) - resid, ffn) < tol


# ------------------------------------------------------------------ fragment-tiled weights
def test_pack_tiled_matches_numpy_order(lib):
    k, n = 256, 48
    w = oracle.normal(52, 2, (k, n), 0.02)
    wd = dev(w)
    dst = torch.empty((n * k,), dtype=torch.int16, device="cuda")
    _abi.check(lib.sfg_hip_pack_weight_v1(wd.data_ptr(), k, n, n, dst.data_ptr(), BF16, 1, stream()))
    q = torch.empty((n * k,), dtype=torch.int8, device="cuda")
    s = torch.empty((n,), dtype=torch.float32, device="cuda")
    _abi.check(lib.sfg_hip_quantize_weight_v1(wd.data_ptr(), k, n, q.data_ptr(), s.data_ptr(), 1, stream()))
    _sync()
    bits = oracle.to_bf16_bits(np.ascontiguousarray(w.T))
    np.testing.assert_array_equal(host(dst).view(np.uint16).reshape(-1), tile_nk(bits, "bf16").reshape(-1))
    qr, sr = oracle.quantize_kn(w)
    np.testing.assert_array_equal(host(q), tile_nk(qr, "int8").reshape(-1))
    np.testing.assert_array_equal(host(s), sr)


@pytest.mark.parametrize("m,n,k", [(16, 3072, 2048), (64, 512, 1024), (7, 256, 384)])
def test_gemm_tiled_integer_operands_exact(lib, m, n, k):
    rng = np.random.default_rng(m * 3 + n)
    a = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
    b = rng.integers(-3, 4, size=(n, k)).astype(np.float32)
    bt = tile_nk(oracle.to_bf16_bits(b), "bf16").view(np.int16)
    c = _gemm(lib, bf16_dev(a), BF16, dev(bt), BF16, m, n, k, EPI_NONE, layout=1)
    np.testing.assert_array_equal(host(c), a @ b.T)
    q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    c8 = _gemm(lib, bf16_dev(a), BF16, dev(tile_nk(q, "int8")), I8, m, n, k, EPI_NONE,
               scales=dev(np.ones(n, np.float32)), layout=1)
    np.testing.assert_array_equal(host(c8), a @ q.astype(np.float32).T)


@pytest.mark.parametrize("epi", [EPI_RESIDUAL, EPI_SWIGLU, EPI_GLU_SILU_UP])
def test_gemm_tiled_epilogues_match_nk(lib, epi):
    m, n, k = 16, 512, 1024
    glu = epi in (EPI_SWIGLU, EPI_GLU_SILU_UP)
    a = oracle.round_bf16(oracle.normal(23, 0, (m, k)))
    b = oracle.normal(23, 2, (2 * n if glu else n, k), 0.02)
    res = oracle.normal(23, 5, (m, n))
    rd = dev(res) if epi == EPI_RESIDUAL else None
    nk = _gemm(lib, bf16_dev(a), BF16, bf16_dev(b), BF16, m, n, k, epi, residual=rd)
    tl = _gemm(lib, bf16_dev(a), BF16, dev(tile_nk(oracle.to_bf16_bits(b), "bf16").view(np.int16)),
               BF16, m, n, k, epi, residual=rd, layout=1)
    # same products, same per-wave k ranges: identical up to summation order inside a wave
    assert oracle.rel_error(host(tl), host(nk)) < 1e-5


def test_gemm_tiled_rejects_prefill_shapes(lib):
    a = torch.zeros((2048, 256), dtype=torch.int16, device="cuda")
    b = torch.zeros((256 * 256,), dtype=torch.int16, device="cuda")
    with pytest.raises(ValueError):
        _gemm(lib, a, BF16, b, BF16, 2048, 256, 256, EPI_NONE, layout=1)


# ------------------------------------------------------------------ target descriptor
def test_target_info_describes_the_device(lib):
    """sfg_hip_target_info_v1 (the GPU counterpart of TargetInfo::detect,
    target.cpp:8-17): queried counts are consistent with each other and with
    torch's view of the device; peaks follow from them."""
    t = _abi.TargetInfo()
    _abi.check(lib.sfg_hip_target_info_v1(0, ctypes.byref(t)))
    arch = t.architecture.decode()
    props = torch.cuda.get_device_properties(0)
    print(f"{arch}: wave {t.wavefront}, {t.compute_units} CUs, {t.xcds} XCDs, LDS {t.lds_bytes_per_cu} B/CU, "
          f"L2 {t.l2_bytes_per_xcd} B/XCD, {t.hbm_bytes >> 30} GiB, {t.engine_clock_ghz:.2f} GHz, "
          f"HBM {t.hbm_gbps:.0f} GB/s, bf16 {t.mfma_bf16_tflops:.0f} TFLOP/s, fp32 {t.valu_fp32_tflops:.1f}")
    assert arch.startswith("gfx950")
    assert t.wavefront == 64 and t.simds_per_cu == 4
    assert t.compute_units == props.multi_processor_count
    assert t.xcds >= 1 and t.compute_units % t.xcds == 0
    assert t.lds_bytes_per_cu == 160 * 1024
    assert t.hbm_bytes == props.total_memory
    assert t.mfma_bf16_tflops == pytest.approx(t.compute_units * 4096 * t.engine_clock_ghz / 1e3)
    assert t.hbm_gbps == 8000.0
    cus, xcds, hbm = ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
    _abi.check(lib.sfg_hip_device_info_v1(0, ctypes.byref(cus), ctypes.byref(xcds), ctypes.byref(hbm)))
    assert (cus.value, xcds.value, hbm.value) == (t.compute_units, t.xcds, t.hbm_bytes)
