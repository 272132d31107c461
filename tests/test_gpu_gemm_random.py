"""Seeded random products through sfg_hip_gemm_v1 and sfg_hip_gemm_grouped_v1
(GPU only), on small-integer operands so that every value is exact.

Dense draws: 1..3000 rows, any width, depths that are and are not multiples
of 32 (the latter on the VALU kernel), bf16 / int8 (power-of-two scales) /
fp32 weights in [N][K] or, for decode rows, fragment-tiled layout, every
epilogue, fp32 or bf16 output, every tile policy, with and without the
split-K workspace.  Grouped draws: 1..8 groups of 0..1200 rows each, gathered
A rows with a few ids outside A (zero rows), bf16 / int8 weights per group.
Expected values: the float64 product of the same operands (exact), its fp32
residual sum, its RNE bf16 rounding for bf16 outputs; GLU epilogues within
2e-5 (fp32 out) or 1e-2 (bf16 out) of the float64 SiLU expression.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from schedforge_amd import _abi
from schedforge_amd._abi import BF16, EPI_GLU_SILU_UP, EPI_NONE, EPI_RESIDUAL, EPI_SWIGLU, F32, I8

from _helpers import KEEP_ALIVE, bf16_dev, dev, host, stream, tile_nk

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEED = 20261204
POW2 = np.array([0.5, 1.0, 2.0], np.float32)


def _epilogue(acc, epi, n, res=None):
    if epi == EPI_NONE:
        return acc
    if epi == EPI_RESIDUAL:
        return acc + res
    g, u = acc[:, :n], acc[:, n:]
    if epi == EPI_SWIGLU:
        return g / (1 + np.exp(np.minimum(-g, 700.0))) * u
    return g * (u / (1 + np.exp(np.minimum(-u, 700.0))))


def _check(c, c_dtype, ref, glu, label):
    if c_dtype == F32:
        if glu:
            np.testing.assert_allclose(host(c), ref, rtol=2e-5, atol=2e-5, err_msg=label)
        else:
            np.testing.assert_array_equal(host(c), ref, err_msg=label)
    else:
        got_bits = host(c).view(np.uint16)
        if glu:
            got = (got_bits.astype(np.uint32) << 16).view(np.float32)
            np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-2, err_msg=label)
        else:
            np.testing.assert_array_equal(got_bits, oracle.to_bf16_bits(ref), err_msg=label)


def _weights(rng, kind, shape, k, layout):
    """(device B, dtype, device scales or None, float64 dequantized B)."""
    if kind == "i8":
        q = rng.integers(-127, 128, size=shape + (k,)).astype(np.int8)
        s = rng.choice(POW2, size=shape).astype(np.float32)
        dq = q.astype(np.float64) * s[..., None]
        return (dev(tile_nk(q, "int8")) if layout else dev(q)), I8, dev(s), dq
    b = rng.integers(-3, 4, size=shape + (k,)).astype(np.float32)
    if kind == "f32":
        return dev(b), F32, None, b.astype(np.float64)
    bd = dev(tile_nk(oracle.to_bf16_bits(b), "bf16").view(np.int16)) if layout else bf16_dev(b)
    return bd, BF16, None, b.astype(np.float64)


def _args(a, a_dtype, b, b_dtype, scales, c, c_dtype, residual, m, n, k, epi, layout, tile):
    g = _abi.GemmArgs()
    g.a, g.a_dtype, g.lda = a.data_ptr(), a_dtype, k
    g.b, g.b_dtype, g.ldb = b.data_ptr(), b_dtype, k
    g.b_scales = scales.data_ptr() if scales is not None else None
    g.c, g.c_dtype, g.ldc = c.data_ptr(), c_dtype, n
    g.residual = residual.data_ptr() if residual is not None else None
    g.ldr = n
    g.m, g.n, g.k, g.epilogue = m, n, k, epi
    g.b_layout, g.tile = layout, tile
    return g


def _dense_case(rng):
    m = int(rng.choice([int(rng.integers(1, 70)), int(rng.integers(70, 3000))]))
    n = int(rng.choice([int(rng.integers(1, 2500)), 16 * int(rng.integers(1, 160)), 128 * int(rng.integers(1, 20))]))
    kc = rng.random()
    k = (32 * int(rng.integers(1, 40)) if kc < 0.5 else
         128 * int(rng.integers(1, 40)) if kc < 0.8 else int(rng.integers(1, 700)))
    epi = int(rng.choice([EPI_NONE, EPI_RESIDUAL, EPI_SWIGLU, EPI_GLU_SILU_UP]))
    glu = epi in (EPI_SWIGLU, EPI_GLU_SILU_UP)
    while m * k * (2 * n if glu else n) > 1.5e9 and k > 32:
        k //= 2
    kind = str(rng.choice(["bf16", "bf16", "i8", "f32"]))
    c_dtype = F32 if (epi == EPI_RESIDUAL or kind == "f32" or rng.random() < 0.5) else BF16
    nb = 2 * n if glu else n
    layout = int(kind != "f32" and m <= 64 and k % 128 == 0 and nb % 16 == 0 and rng.random() < 0.5)
    return dict(m=m, n=n, k=k, epi=epi, kind=kind, c_dtype=c_dtype, layout=layout,
                tile=int(rng.integers(0, _abi.TILE_COUNT)), workspace=bool(rng.random() < 0.7))


def _grouped_case(rng):
    groups = int(rng.integers(1, 9))
    counts = [int(rng.choice([0, int(rng.integers(1, 40)), int(rng.integers(40, 1200))])) for _ in range(groups)]
    if sum(counts) == 0:
        counts[0] = 5
    n = int(rng.choice([16 * int(rng.integers(1, 80)), int(rng.integers(1, 900))]))
    k = 32 * int(rng.integers(1, 40)) if rng.random() < 0.7 else 128 * int(rng.integers(1, 20))
    epi = int(rng.choice([EPI_NONE, EPI_SWIGLU, EPI_GLU_SILU_UP]))
    while sum(counts) * k * (2 * n if epi != EPI_NONE else n) > 1.5e9 and k > 32:
        k //= 2
    return dict(counts=counts, n=n, k=k, epi=epi, kind=str(rng.choice(["bf16", "i8"])),
                c_dtype=F32 if rng.random() < 0.5 else BF16, a_rows=int(rng.integers(1, 1200)),
                tile=int(rng.integers(0, _abi.TILE_COUNT)))


def _cases(n=40):
    rng = np.random.default_rng(SEED)
    return [("grouped", _grouped_case(rng)) if rng.random() < 0.4 else ("dense", _dense_case(rng))
            for _ in range(n)]


CASES = _cases()


@pytest.mark.parametrize("idx", range(len(CASES)), ids=[f"{c[0]}{i}" for i, c in enumerate(CASES)])
def test_random_product_is_exact(idx):
    lib = _abi.load()
    kind_of_case, c = CASES[idx]
    label = f"{kind_of_case} {c}"
    print(label, flush=True)
    rng = np.random.default_rng(SEED + idx)
    glu = c["epi"] in (EPI_SWIGLU, EPI_GLU_SILU_UP)
    n, k = c["n"], c["k"]
    nb = 2 * n if glu else n
    if kind_of_case == "dense":
        m = c["m"]
        a = rng.integers(-3, 4, size=(m, k)).astype(np.float32)
        res = rng.integers(-5, 6, size=(m, n)).astype(np.float32)
        bd, b_dtype, sd, bm = _weights(rng, c["kind"], (nb,), k, c["layout"])
        ad, a_dtype = (dev(a), F32) if c["kind"] == "f32" else (bf16_dev(a), BF16)
        rd = dev(res) if c["epi"] == EPI_RESIDUAL else None
        out = torch.empty((m, n), dtype=torch.float32 if c["c_dtype"] == F32 else torch.int16, device="cuda")
        KEEP_ALIVE.append(out)
        args = _args(ad, a_dtype, bd, b_dtype, sd, out, c["c_dtype"], rd, m, n, k, c["epi"], c["layout"], c["tile"])
        if c["workspace"]:
            ws = torch.zeros(max(lib.sfg_hip_gemm_workspace_v1(m, n, k), 256), dtype=torch.uint8, device="cuda")
            KEEP_ALIVE.append(ws)
            _abi.check(lib.sfg_hip_gemm_v1(ctypes.byref(args), ws.data_ptr(), ws.numel(), stream()))
        else:
            _abi.check(lib.sfg_hip_gemm_v1(ctypes.byref(args), None, 0, stream()))
        torch.cuda.synchronize()
        acc = a.astype(np.float64) @ bm.T
        _check(out, c["c_dtype"], _epilogue(acc, c["epi"], n, res).astype(np.float32), glu, label)
        return
    counts, T = c["counts"], c["a_rows"]
    groups, m = len(counts), sum(counts)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    a = rng.integers(-3, 4, size=(T, k)).astype(np.float32)
    rows = rng.integers(0, T, size=m).astype(np.int32)
    outside = rng.random(m) < 0.03
    rows[outside] = np.where(rng.random(int(outside.sum())) < 0.5, -1, T + 3)
    bd, b_dtype, sd, bm = _weights(rng, c["kind"], (groups, nb), k, 0)
    out = torch.empty((m, n), dtype=torch.float32 if c["c_dtype"] == F32 else torch.int16, device="cuda")
    ws = torch.zeros(max(lib.sfg_hip_gemm_workspace_v1(m, n, k), 256), dtype=torch.uint8, device="cuda")
    KEEP_ALIVE.extend([out, ws])
    args = _args(bf16_dev(a), BF16, bd, b_dtype, sd, out, c["c_dtype"], None, m, n, k, c["epi"], 0, c["tile"])
    _abi.check(lib.sfg_hip_gemm_grouped_v1(ctypes.byref(args), dev(rows).data_ptr(), T,
                                           dev(offsets).data_ptr(), groups, nb * k,
                                           nb if sd is not None else 0, ws.data_ptr(), ws.numel(),
                                           stream()))
    torch.cuda.synchronize()
    acc = np.zeros((m, nb))
    for g in range(groups):
        src = rows[offsets[g]:offsets[g + 1]]
        valid = (src >= 0) & (src < T)
        arow = np.zeros((len(src), k))
        arow[valid] = a[src[valid]]
        acc[offsets[g]:offsets[g + 1]] = arow @ bm[g].T
    _check(out, c["c_dtype"], _epilogue(acc, c["epi"], n).astype(np.float32), glu, label)
