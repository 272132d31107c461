"""Seeded random paged attention through the two C-ABI entry points (GPU only).

sfg_hip_attn_paged_v1 (any head_dim up to 256, any page size, 1..8 new rows
per sequence under the causal offset j <= L - S + i of attention_compiler.cpp:
68-72, or none, fp32 or bf16 pools) and sfg_hip_attn_decode_paged_v1 (bf16
pools, one new token; head_dim 64 / 128 over 16-token pages run the MFMA split
kernel) on draws the hand-picked tests do not make: ragged lengths with a
sequence of length 0, no device lengths (every sequence reads max_context
keys), page tables with unused trailing entries, pools with pages no table
names and stale contents everywhere else, and split counts from 1 to 64
(more splits than pages included).  The expected output is the definition --
softmax of the scaled dot products over the visible keys, in float64 on the
same (bf16-rounded) operands -- and a row with no visible key is NaN, the
reference's 0 / 0.  Tolerance (max |got - ref| / max |ref| over the finite
rows): 1e-4 for the fp32 row kernel, 2e-2 for the MFMA kernel's bf16
operands.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle

from _helpers import KEEP_ALIVE, dev

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEED = 20261203


def _expected(q, k, v, lens, causal, scale):
    B, Hq, S, D = q.shape
    group = Hq // k.shape[1]
    out = np.full((B, Hq, S, D), np.nan)
    for b in range(B):
        L = lens[b]
        for h in range(Hq):
            kk = k[b, h // group, :L].astype(np.float64)
            vv = v[b, h // group, :L].astype(np.float64)
            s = q[b, h].astype(np.float64) @ kk.T * scale
            if causal:
                s = np.where(np.arange(L)[None, :] <= L - S + np.arange(S)[:, None], s, -np.inf)
            for r in range(S):
                if np.isfinite(s[r]).any():
                    p = np.exp(s[r] - s[r].max())
                    out[b, h, r] = p @ vv / p.sum()
    return out


def _pools(rng, B, Hkv, lens, D, pt, pps, bf16):
    L = max(max(lens), 1)
    k = rng.standard_normal((B, Hkv, L, D)).astype(np.float32)
    v = rng.standard_normal((B, Hkv, L, D)).astype(np.float32)
    if bf16:
        k, v = oracle.round_bf16(k), oracle.round_bf16(v)
    pages = B * pps + int(rng.integers(0, 5))
    table = rng.permutation(pages)[:B * pps].astype(np.int32).reshape(B, pps)
    kp = rng.standard_normal((pages, Hkv, pt, D)).astype(np.float32)   # stale contents
    vp = rng.standard_normal((pages, Hkv, D, pt)).astype(np.float32)
    for b in range(B):
        for t in range(lens[b]):
            kp[table[b, t // pt], :, t % pt, :] = k[b, :, t, :]
            vp[table[b, t // pt], :, :, t % pt] = v[b, :, t, :]
    return k, v, kp, vp, table, pages


def _draw(rng):
    mfma = bool(rng.random() < 0.4)
    if mfma:
        D, pt, S, bf16 = int(rng.choice([64, 128])), 16, 1, True
        Hkv, group = int(rng.choice([1, 2, 4, 8])), int(rng.choice([1, 2, 4, 8, 16]))
    else:
        D = int(rng.choice([1, 2, 4, 7, 8, 16, 33, 64, 96, 128, 160, 256]))
        pt = int(rng.choice([1, 2, 3, 4, 8, 16, 32, 64]))
        S = int(rng.choice([1, 1, 2, 3, 5, 8]))
        bf16 = bool(rng.random() < 0.5)
        Hkv, group = int(rng.choice([1, 2, 3, 4])), int(rng.choice([1, 2, 3, 4, 8, 32]))
    B = int(rng.integers(2, 24 if not mfma else 40))
    maxc = int(rng.choice([int(rng.integers(1, 40)), int(rng.integers(40, 1500))]))
    causal = 1 if (mfma or rng.random() < 0.8) else 0
    if causal:
        maxc = max(maxc, S)
    lens = [int(rng.integers(1, maxc + 1)) for _ in range(B)]
    lens[int(rng.integers(0, B))] = maxc
    if rng.random() < 0.5:
        lens[int(rng.integers(0, B))] = 0
    return dict(mfma=mfma, D=D, pt=pt, S=S, bf16=bf16, Hkv=Hkv, Hq=Hkv * group, B=B, maxc=maxc,
                causal=causal, lens=lens, pps=(maxc + pt - 1) // pt + int(rng.integers(0, 3)),
                splits=int(rng.choice([0, 0, 1, 2, 3, 7, 16, 64])),
                scale=float(rng.choice([0.0, 0.3])), device_lens=bool(rng.random() < 0.8))


def _cases(n=24):
    rng = np.random.default_rng(SEED)
    return [(_draw(rng), SEED + i) for i in range(n)]


CASES = _cases()


@pytest.mark.parametrize("idx", range(len(CASES)), ids=[f"case{i}" for i in range(len(CASES))])
def test_random_paged_attention_matches_the_definition(idx):
    from schedforge_amd import _abi
    lib = _abi.load()
    c, seed = CASES[idx]
    rng = np.random.default_rng(seed)
    B, Hq, Hkv, S, D, pt, pps, maxc = (c[x] for x in ("B", "Hq", "Hkv", "S", "D", "pt", "pps", "maxc"))
    label = ", ".join(f"{k}={v}" for k, v in c.items() if k != "lens")
    print(label, flush=True)
    eff = c["lens"] if c["device_lens"] else [maxc] * B   # no device lengths: max_context keys each
    k, v, kp, vp, table, pages = _pools(rng, B, Hkv, eff, D, pt, pps, c["bf16"])
    q = rng.standard_normal((B, Hq, S, D)).astype(np.float32)
    scale = c["scale"] if c["scale"] > 0 else 1.0 / np.sqrt(D)
    ref = _expected(q, k, v, eff, c["causal"], scale)
    if c["bf16"]:
        kpd = dev(oracle.to_bf16_bits(kp).view(np.int16))
        vpd = dev(oracle.to_bf16_bits(vp).view(np.int16))
        kvdt = _abi.BF16
    else:
        kpd, vpd, kvdt = dev(kp), dev(vp), _abi.F32
    tab = dev(table)
    lens_ptr = dev(np.asarray(eff, np.int32)).data_ptr() if c["device_lens"] else None
    if c["mfma"]:
        out = torch.empty((B, Hq * D), dtype=torch.float32, device="cuda")
        wsb = lib.sfg_hip_attn_decode_workspace_v1(B, Hq, D, maxc, pt, c["splits"])
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
        KEEP_ALIVE.extend([out, ws])
        _abi.check(lib.sfg_hip_attn_decode_paged_v1(
            dev(np.ascontiguousarray(q[:, :, 0, :])).data_ptr(), kpd.data_ptr(), vpd.data_ptr(),
            tab.data_ptr(), lens_ptr, out.data_ptr(), _abi.F32, B, Hq, Hkv, D, pt, pps, pages, maxc,
            c["splits"], ctypes.c_float(c["scale"]), 1, ws.data_ptr(), ws.numel(), None))
        got = out.cpu().numpy().reshape(B, Hq, 1, D)
        tol = 2e-2
    else:
        out = torch.empty((B, Hq, S, D), dtype=torch.float32, device="cuda")
        wsb = lib.sfg_hip_attn_paged_workspace_v1(B, Hq, Hkv, S, D, kvdt, maxc, pt, c["splits"])
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
        KEEP_ALIVE.extend([out, ws])
        _abi.check(lib.sfg_hip_attn_paged_v1(
            dev(q).data_ptr(), kpd.data_ptr(), vpd.data_ptr(), kvdt, tab.data_ptr(), lens_ptr,
            out.data_ptr(), _abi.F32, B, Hq, Hkv, S, D, pt, pps, pages, maxc, c["causal"],
            c["splits"], ctypes.c_float(c["scale"]), 1, ws.data_ptr(), ws.numel(), None))
        got = out.cpu().numpy()
        tol = 1e-4
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref), err_msg=label)
    finite = ~np.isnan(ref)
    if finite.any():
        err = np.abs(got[finite] - ref[finite]).max() / np.abs(ref[finite]).max()
        assert err < tol, (label, err)
