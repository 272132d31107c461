"""sfg_hip_attn_decode_paged_noalloc_v1 (GPU only): the paged Split-KV decode
with its split partials in the library's device scratch array instead of a
caller workspace, called through the C ABI.  Its output must equal, bit for bit,
sfg_hip_attn_decode_paged_v1's with the same split count, on two calls in a row
(the second smaller, so stale partials of the first would show), bf16 and fp32
outputs, on the MFMA kernel's shapes and on the row kernel's; captured into a
HIP graph after an eager first call, every replay matches too; a request whose
partials exceed the array is refused before any launch.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from schedforge_amd import _abi

from _helpers import bf16_dev, dev, host, stream

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

PT, D = 16, 128


def _case(B, Hq, Hkv, ctx, seed):
    pps = (ctx + PT - 1) // PT
    num_pages = B * pps + 5
    table = oracle.page_permutation(seed, num_pages)[: B * pps].reshape(B, pps).astype(np.int32)
    kc = oracle.round_bf16(oracle.normal(seed, 15, (B, Hkv, ctx, D)))
    vc = oracle.round_bf16(oracle.normal(seed, 16, (B, Hkv, ctx, D)))
    kp = oracle.paged_scatter(kc, table, num_pages, PT)
    vp = np.ascontiguousarray(oracle.paged_scatter(vc, table, num_pages, PT).transpose(0, 1, 3, 2))
    lens = np.random.default_rng(seed).integers(1, ctx + 1, size=B).astype(np.int32)
    lens[0] = ctx
    return dict(q=dev(oracle.normal(seed, 0, (B, Hq, 1, D))), k=bf16_dev(kp), v=bf16_dev(vp),
                table=dev(table), lens=dev(lens), B=B, Hq=Hq, Hkv=Hkv, ctx=ctx, pps=pps,
                num_pages=num_pages)


def _args(c):
    return (c["q"].data_ptr(), c["k"].data_ptr(), c["v"].data_ptr(), c["table"].data_ptr(),
            c["lens"].data_ptr())


def _dims(c, splits):
    return (c["B"], c["Hq"], c["Hkv"], D, PT, c["pps"], c["num_pages"], c["ctx"], splits,
            ctypes.c_float(0.0))


def _with_workspace(lib, c, out_dtype, splits):
    tdt = torch.float32 if out_dtype == _abi.F32 else torch.int16
    out = torch.empty((c["B"], c["Hq"] * D), dtype=tdt, device="cuda")
    wsb = lib.sfg_hip_attn_decode_workspace_v1(c["B"], c["Hq"], D, c["ctx"], PT, splits)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    _abi.check(lib.sfg_hip_attn_decode_paged_v1(*_args(c), out.data_ptr(), out_dtype,
                                                *_dims(c, splits), 0, ws.data_ptr(), ws.numel(),
                                                stream()))
    torch.cuda.synchronize()
    return host(out)


def _no_alloc(lib, c, out_dtype, splits):
    tdt = torch.float32 if out_dtype == _abi.F32 else torch.int16
    out = torch.empty((c["B"], c["Hq"] * D), dtype=tdt, device="cuda")
    _abi.check(lib.sfg_hip_attn_decode_paged_noalloc_v1(*_args(c), out.data_ptr(), out_dtype,
                                                        *_dims(c, splits), stream()))
    torch.cuda.synchronize()
    return host(out)


@pytest.mark.parametrize("out_dtype", [_abi.F32, _abi.BF16])
def test_no_alloc_decode_matches_workspace_entry_twice(out_dtype):
    lib = _abi.load()
    big = _case(16, 16, 4, 4096, 601)       # C2's attention shape, ragged lengths
    small = _case(3, 8, 2, 700, 602)        # then a smaller call on the same scratch
    for c, splits in ((big, 0), (small, 0), (big, 8), (small, 3)):
        want = _with_workspace(lib, c, out_dtype, splits)
        got = _no_alloc(lib, c, out_dtype, splits)
        print(f"B{c['B']} Hq{c['Hq']} ctx{c['ctx']} splits {splits}: equal {np.array_equal(got, want)}")
        np.testing.assert_array_equal(got, want)
        if out_dtype == _abi.F32:
            assert np.isfinite(got).all()


def test_no_alloc_decode_refuses_partials_beyond_the_scratch():
    """64 sequences x 64 heads x 8 splits x (128 + 2) x 4 B = 17 MB > 16 MiB:
    SFG_ERR_WORKSPACE before any launch (the pointers are never read)."""
    lib = _abi.load()
    c = _case(1, 8, 2, 64, 603)
    B, Hq, Hkv, ctx, splits = 64, 64, 8, 8192, 8
    need = lib.sfg_hip_attn_decode_workspace_v1(B, Hq, D, ctx, PT, splits)
    assert need > 16 << 20
    out = torch.empty(16, dtype=torch.float32, device="cuda")
    rc = lib.sfg_hip_attn_decode_paged_noalloc_v1(*_args(c), out.data_ptr(), _abi.F32, B, Hq, Hkv,
                                                  D, PT, ctx // PT, B * ctx // PT, ctx, splits,
                                                  ctypes.c_float(0.0), stream())
    assert rc == _abi.ERR_WORKSPACE
    assert b"scratch" in lib.sfg_hip_last_error()


def test_no_alloc_decode_replays_under_graph_capture():
    """After a first eager call on the device (which looks the scratch address
    up, outside any capture), the entry point captures into a HIP graph: it
    records kernel launches only.  Each of three replays, with new query values
    copied in eagerly and the stream synchronised between them, equals the
    workspace entry point on the same inputs bit for bit."""
    lib = _abi.load()
    c = _case(8, 16, 4, 1024, 604)
    _no_alloc(lib, c, _abi.F32, 0)  # warm-up on this device, eager
    out = torch.empty((c["B"], c["Hq"] * D), dtype=torch.float32, device="cuda")
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=side):
        rc = lib.sfg_hip_attn_decode_paged_noalloc_v1(*_args(c), out.data_ptr(), _abi.F32,
                                                      *_dims(c, 0), side.cuda_stream)
    assert rc == 0, lib.sfg_hip_last_error()
    for rep in range(3):
        c["q"].copy_(torch.from_numpy(oracle.normal(700 + rep, 0, (c["B"], c["Hq"], 1, D))))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = host(out)
        want = _with_workspace(lib, c, _abi.F32, 0)
        print(f"replay {rep}: equal {np.array_equal(got, want)}")
        np.testing.assert_array_equal(got, want)


def test_no_alloc_decode_on_the_row_kernel_matches_workspace_entry():
    """A shape the MFMA split kernel does not lower (head_dim 96, 8-token
    pages) runs the row kernel with its partials in the same scratch, bit for
    bit equal to the workspace entry point, twice in a row with different
    split counts."""
    lib = _abi.load()
    B, Hq, Hkv, d, pt, ctx, seed = 3, 6, 2, 96, 8, 300, 605
    pps = (ctx + pt - 1) // pt
    table = oracle.page_permutation(seed, B * pps).reshape(B, pps).astype(np.int32)
    kp = oracle.round_bf16(oracle.normal(seed, 15, (B * pps, Hkv, pt, d)))
    vp = oracle.round_bf16(oracle.normal(seed, 16, (B * pps, Hkv, d, pt)))
    q, k, v = dev(oracle.normal(seed, 0, (B, Hq, 1, d))), bf16_dev(kp), bf16_dev(vp)
    tab, lens = dev(table), dev(np.array([ctx, 17, 123], np.int32))
    for splits in (4, 0):
        outs = []
        for noalloc in (False, True):
            out = torch.empty((B, Hq * d), dtype=torch.float32, device="cuda")
            args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), tab.data_ptr(), lens.data_ptr(),
                    out.data_ptr(), _abi.F32, B, Hq, Hkv, d, pt, pps, B * pps, ctx, splits,
                    ctypes.c_float(0.0))
            if noalloc:
                _abi.check(lib.sfg_hip_attn_decode_paged_noalloc_v1(*args, stream()))
            else:
                wsb = lib.sfg_hip_attn_decode_workspace_v1(B, Hq, d, ctx, pt, splits)
                ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device="cuda")
                _abi.check(lib.sfg_hip_attn_decode_paged_v1(*args, 1, ws.data_ptr(), ws.numel(), stream()))
            torch.cuda.synchronize()
            outs.append(host(out))
        np.testing.assert_array_equal(outs[1], outs[0])
        assert np.isfinite(outs[0]).all()
