"""C-ABI checks that need no GPU: the library loads, exports every entry point
include/sfg_hip.h declares, and rejects invalid arguments on the host with the
reference's error classes (codes < 16 -> ValueError, the reference's
std::invalid_argument; validate() at decoder_compiler.cpp:26-39)."""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from schedforge_amd import _abi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sfg_hip.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|size_t|const char\*)\s+(sfg_hip_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    return _abi.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared_functions()
    assert len(names) >= 25
    out = subprocess.run(["nm", "-D", "--defined-only", str(_abi.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (sfg_hip_\w+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    # and the Python binding covers exactly the declared surface
    assert sorted(_abi.EXPORTED) == names


def test_no_undefined_library_symbols():
    """Every kernel's host launch stub is defined (a kernel whose host-side
    instantiation fails leaves an undefined stub that only an eager load sees)."""
    out = subprocess.run(["nm", "-D", "--undefined-only", str(_abi.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    undefined = [l for l in out.splitlines() if "sfg" in l]
    assert not undefined, undefined[:5]


def test_identity(lib):
    assert lib.sfg_hip_abi_version() == _abi.ABI_VERSION
    meta = lib.sfg_hip_metadata_v1().decode()
    assert "abi=1" in meta and "arch=gfx950" in meta


def _desc(**kw):
    d = _abi.LayerDesc()
    d.abi = _abi.ABI_VERSION
    base = dict(batch=2, sequence=1, hidden=256, intermediate=512, query_heads=2, kv_heads=1,
                head_dim=128, rms_epsilon=1e-5, rope_theta=1e4, causal=1, ffn=0, experts=4, top_k=2,
                context=64, page_tokens=16, pages_per_seq=4, num_pages=8, act_dtype=_abi.BF16,
                weight_dtype=_abi.BF16, kv_splits=0, use_routing_trace=0)
    base.update(kw)
    for k, v in base.items():
        setattr(d, k, v)
    return d


def _call_layer(lib, d):
    io = _abi.LayerIO()
    w = _abi.LayerWeights()
    return lib.sfg_hip_decoder_layer_v1(ctypes.byref(d), ctypes.byref(w), ctypes.byref(io), None, 0, None)


def test_workspace_query_and_validation(lib):
    assert lib.sfg_hip_decoder_layer_workspace_v1(ctypes.byref(_desc())) > 0
    for bad in (dict(hidden=250), dict(kv_heads=3, query_heads=2), dict(rms_epsilon=0.0),
                dict(ffn=1, top_k=5), dict(context=-1)):
        d = _desc(**bad)
        assert lib.sfg_hip_decoder_layer_workspace_v1(ctypes.byref(d)) == 0
        assert _call_layer(lib, d) == _abi.ERR_INVALID_CONFIG, bad


def test_abi_mismatch_and_guards(lib):
    d = _desc()
    d.abi = 99
    assert _call_layer(lib, d) == _abi.ERR_ABI
    # context beyond the plan's page capacity: compiled guard
    assert _call_layer(lib, _desc(context=65)) == _abi.ERR_GUARD
    # fp32 activations with int8 weights are not lowered
    assert _call_layer(lib, _desc(act_dtype=_abi.F32, weight_dtype=_abi.I8, context=0)) == _abi.ERR_UNSUPPORTED
    # missing weights / io
    assert _call_layer(lib, _desc()) == _abi.ERR_SHAPE
    with pytest.raises(ValueError, match="null weights or io"):
        _abi.check(_call_layer(lib, _desc()))


def test_op_entry_points_validate_on_host(lib):
    args = _abi.GemmArgs()
    assert lib.sfg_hip_gemm_v1(ctypes.byref(args), None, 0, None) == _abi.ERR_SHAPE
    assert lib.sfg_hip_rmsnorm_v1(None, None, None, _abi.F32, 0, 0, ctypes.c_float(1e-5), None) == _abi.ERR_SHAPE
    # causal attention with Sq > Skv (attention_compiler.cpp:23-29)
    rc = lib.sfg_hip_attn_prefill_v1(1, 1, 1, 1, _abi.BF16, _abi.BF16, 1, 2, 1, 8, 4, 128, 1,
                                     ctypes.c_float(0.0), None)
    assert rc == _abi.ERR_INVALID_CONFIG
    # flash prefill over V^T: keys padded to 64, head_dim 128 only
    assert [lib.sfg_hip_attn_vt_ld_v1(s) for s in (1, 64, 65, 8192)] == [64, 64, 128, 8192]
    rc = lib.sfg_hip_attn_prefill_vt_v1(1, 1, 1, 100, 1, _abi.F32, 1, 2, 1, 100, 100, 128, 1,
                                        ctypes.c_float(0.0), None)
    assert rc == _abi.ERR_SHAPE  # ld_vt must be 128 for 100 keys
    rc = lib.sfg_hip_attn_prefill_vt_v1(1, 1, 1, 128, 1, _abi.F32, 1, 2, 1, 100, 100, 64, 1,
                                        ctypes.c_float(0.0), None)
    assert rc == _abi.ERR_UNSUPPORTED  # head_dim 64
    rc = lib.sfg_hip_attn_prefill_vt_v1(1, 1, 1, 64, 1, _abi.F32, 1, 2, 1, 8, 4, 128, 1,
                                        ctypes.c_float(0.0), None)
    assert rc == _abi.ERR_INVALID_CONFIG
    rc = lib.sfg_hip_qkv_split_rope_vt_v1(1, 1, 1, 8, 2, 1, 64, 1, 1, 1, 64, None)
    assert rc == _abi.ERR_UNSUPPORTED
    # paged decode: context beyond the page table (guard) and bad GQA ratio (config)
    rc = lib.sfg_hip_attn_decode_paged_v1(1, 1, 1, 1, None, 1, _abi.F32, 1, 4, 1, 128, 16, 2, 2, 33,
                                          0, ctypes.c_float(0.0), 0, None, 0, None)
    assert rc == _abi.ERR_GUARD
    rc = lib.sfg_hip_attn_decode_paged_v1(1, 1, 1, 1, None, 1, _abi.F32, 1, 4, 3, 128, 16, 2, 2, 32,
                                          0, ctypes.c_float(0.0), 0, None, 0, None)
    assert rc == _abi.ERR_INVALID_CONFIG
    # MoE: top_k > experts (moe_compiler.cpp:41-45)
    rc = lib.sfg_hip_moe_route_v1(1, 1, None, 4, 8, 2, 3, 1, 1, 1, 1, 1, 1, 1, 1, None, 0, None)
    assert rc == _abi.ERR_INVALID_CONFIG
    msg = lib.sfg_hip_last_error().decode()
    assert "MoE" in msg


def test_rope_table_matches_reference_expressions(lib):
    seq, d, theta = 5, 16, 10000.0
    t = np.empty((seq, d // 2, 2), np.float32)
    assert lib.sfg_hip_rope_table_host_v1(t.ctypes.data, seq, d, ctypes.c_float(theta)) == 0
    i = np.arange(0, d, 2, dtype=np.float32)
    f = np.power(np.float32(theta), -i / np.float32(d)).astype(np.float32)
    ang = (np.arange(seq, dtype=np.float32)[:, None] * f[None, :]).astype(np.float32)
    np.testing.assert_allclose(t[..., 0], np.cos(ang.astype(np.float64)), atol=2e-7)
    np.testing.assert_allclose(t[..., 1], np.sin(ang.astype(np.float64)), atol=2e-7)
    np.testing.assert_array_equal(t[0, :, 0], 1.0)
    np.testing.assert_array_equal(t[0, :, 1], 0.0)


def test_layer_taps_lie_inside_the_workspace(lib):
    """sfg_hip_decoder_layer_tap_v1 (host-only query): every stage tap is a
    distinct region inside the layer workspace, with its documented size and
    dtype; routing taps exist only for a MoE layer routed on the device."""
    def tap(d, t):
        off, nb, dt = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_int()
        rc = lib.sfg_hip_decoder_layer_tap_v1(ctypes.byref(d), t, ctypes.byref(off), ctypes.byref(nb),
                                              ctypes.byref(dt))
        return rc, off.value, nb.value, dt.value
    for kw in (dict(), dict(context=0, sequence=64), dict(ffn=1), dict(ffn=1, use_routing_trace=1)):
        d = _desc(**kw)
        ws = lib.sfg_hip_decoder_layer_workspace_v1(ctypes.byref(d))
        rows, H, k = d.batch * d.sequence, d.hidden, d.top_k
        expect = {_abi.TAP_ATTN: (rows * H * 2, _abi.BF16), _abi.TAP_RESIDUAL1: (rows * H * 4, _abi.F32),
                  _abi.TAP_NORM2: (rows * H * 2, _abi.BF16)}
        if d.ffn == 1:
            expect[_abi.TAP_ROUTE_INPUT] = (rows * H * 4, _abi.F32)
        if d.ffn == 1 and not d.use_routing_trace:
            expect[_abi.TAP_ROUTE_IDS] = (rows * k * 4, _abi.I32)
            expect[_abi.TAP_ROUTE_WEIGHTS] = (rows * k * 4, _abi.F32)
        spans = []
        for t in range(_abi.NUM_TAPS):
            rc, off, nb, dt = tap(d, t)
            if t not in expect:
                assert rc == _abi.ERR_UNSUPPORTED, (kw, t)
                continue
            assert rc == 0 and (nb, dt) == expect[t], (kw, t, nb, dt)
            assert off % 256 == 0 and off + nb <= ws
            spans.append((off, off + nb))
        spans.sort()
        assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:])), spans
    assert tap(_desc(), 99)[0] == _abi.ERR_SHAPE
    assert tap(_desc(hidden=250), 0)[0] == _abi.ERR_INVALID_CONFIG


def test_random_descriptors_get_a_code_and_a_sane_workspace(lib):
    """3000 seeded descriptors with fields drawn from edge values (0, -1,
    2^31 - 1, mismatched head counts, unknown dtypes, layouts, tile and wave
    policies): the workspace query and the layer entry (null weights / io)
    return an ABI code, never crash; every descriptor the query accepts reports
    at least the bf16 bytes of its activation rows (no 32-bit wrap)."""
    rng = np.random.default_rng(20261205)
    i32 = 2**31 - 1
    edge = [0, 1, -1, 2, 3, 7, 16, 64, 128, 1000, 4096, 65536, 1 << 20, i32, -i32 - 1]
    codes = {_abi.ERR_INVALID_CONFIG, _abi.ERR_SHAPE, _abi.ERR_UNSUPPORTED, _abi.ERR_GUARD}
    pick = lambda xs: int(rng.choice(xs))
    for _ in range(3000):
        d = _abi.LayerDesc()
        d.abi = _abi.ABI_VERSION
        d.head_dim = pick([1, 4, 64, 128, 256, 257, 0, -4, 1 << 16])
        d.query_heads = pick([1, 2, 8, 32, 128, 0, -1, 1 << 12])
        d.kv_heads = pick([1, 2, 4, 8, 3, 0])
        d.hidden = d.query_heads * d.head_dim if rng.random() < 0.8 else pick(edge)
        d.batch, d.sequence, d.intermediate, d.context = (pick(edge) for _ in range(4))
        d.pages_per_seq, d.num_pages = pick(edge), pick(edge)
        d.page_tokens = pick([0, 1, 16, -16, 1 << 20])
        d.rms_epsilon = float(rng.choice([1e-6, 0.0, -1.0, float("nan")]))
        d.rope_theta, d.causal, d.ffn = 1e4, pick([0, 1]), pick([0, 1, 2])
        d.experts, d.top_k = pick([0, 1, 8, 64, -1, 4096]), pick([0, 1, 2, 8, 9])
        d.act_dtype = pick([_abi.F32, _abi.BF16, 7])
        d.weight_dtype = pick([_abi.F32, _abi.BF16, _abi.I8, 9])
        d.kv_splits, d.use_routing_trace = pick([0, 1, 64, -3, i32]), pick([0, 1])
        d.weight_layout, d.kv_append = pick([0, 1, 5]), pick([0, 1])
        d.gemm_tile, d.attn_waves = pick([0, 3, 8, -1]), pick([0, 4, 8, 5])
        ws = lib.sfg_hip_decoder_layer_workspace_v1(ctypes.byref(d))
        rc = lib.sfg_hip_decoder_layer_v1(ctypes.byref(d), ctypes.byref(_abi.LayerWeights()),
                                          ctypes.byref(_abi.LayerIO()), None, 0, None)
        assert rc in codes, rc
        if ws:
            assert ws >= d.batch * d.sequence * d.hidden * 2


def test_widened_layer_domain_validates_on_host(lib):
    """Decode on fp32 pools, MoE on fp32 activations, several new tokens per
    decode step and head dims up to 256 are lowered (a workspace size comes
    back); a causal step longer than its cache (validate_config,
    attention_compiler.cpp:23-29) and head dims above 256 are refused."""
    ws = lambda **kw: lib.sfg_hip_decoder_layer_workspace_v1(ctypes.byref(_desc(**kw)))
    assert ws(act_dtype=_abi.F32, weight_dtype=_abi.F32) > 0                       # fp32 decode
    assert ws(act_dtype=_abi.F32, weight_dtype=_abi.F32, ffn=1, context=0) > 0      # fp32 MoE
    assert ws(sequence=3) > 0                                                        # S = 3 decode
    assert ws(hidden=8, query_heads=2, head_dim=4, page_tokens=4, pages_per_seq=16, num_pages=32) > 0
    assert ws(sequence=3, kv_append=1, context=61) > 0                               # append 3
    assert _call_layer(lib, _desc(sequence=65)) == _abi.ERR_INVALID_CONFIG          # S > context
    assert _call_layer(lib, _desc(sequence=4, kv_append=1, context=61)) == _abi.ERR_GUARD  # past capacity
    assert _call_layer(lib, _desc(hidden=2 * 320, head_dim=320, context=0)) == _abi.ERR_UNSUPPORTED


def test_generic_paged_attention_entry_validates_on_host(lib):
    """sfg_hip_attn_paged_v1 rejects on the host, before any launch."""
    call = lambda **kw: lib.sfg_hip_attn_paged_v1(
        *[kw.get(k, v) for k, v in dict(
            q=1, k=1, v=1, kv_dtype=_abi.F32, table=1, lens=None, out=1, out_dtype=_abi.F32, batch=1,
            hq=4, hkv=2, sq=1, d=4, pt=4, pps=3, pages=3, ctx=7, causal=1, splits=0).items()],
        ctypes.c_float(0.0), 0, None, kw.get("ws_bytes", 0), None)
    assert call(sq=8) == _abi.ERR_INVALID_CONFIG        # causal, 8 rows over 7 keys
    assert call(d=257) == _abi.ERR_UNSUPPORTED          # head_dim above 256
    assert call(kv_dtype=_abi.I8) == _abi.ERR_UNSUPPORTED
    assert call(ctx=13) == _abi.ERR_GUARD               # beyond 3 pages of 4 tokens
    assert call(hkv=3) == _abi.ERR_INVALID_CONFIG       # GQA ratio
    # several splits need a workspace
    need = lib.sfg_hip_attn_paged_workspace_v1(1, 4, 2, 1, 4, _abi.F32, 7, 4, 3)
    assert need > 0 and call(splits=3) == _abi.ERR_WORKSPACE
    # the bf16 decode entry's workspace query bounds the general one from above
    # (it assumes the worst kv_heads and covers both kernels)
    for hkv in (1, 4, 16):
        assert 0 < lib.sfg_hip_attn_paged_workspace_v1(16, 16, hkv, 1, 128, _abi.BF16, 4096, 16, 0) <= \
            lib.sfg_hip_attn_decode_workspace_v1(16, 16, 128, 4096, 16, 0)


def test_grouped_gemm_and_pool_entries_validate_on_host(lib):
    args = _abi.GemmArgs()
    args.a = args.b = args.c = 1
    args.m, args.n, args.k, args.lda, args.ldb, args.ldc = 8, 8, 8, 8, 8, 8
    args.epilogue = 1  # SFG_EPI_RESIDUAL: no residual in the grouped form
    assert lib.sfg_hip_gemm_grouped_v1(ctypes.byref(args), None, 0, 1, 2, 0, 0, None, 0, None) == _abi.ERR_SHAPE
    args.epilogue = 0
    assert lib.sfg_hip_gemm_grouped_v1(ctypes.byref(args), None, 0, None, 2, 0, 0, None, 0, None) == _abi.ERR_SHAPE
    assert lib.sfg_hip_kv_append_pool_v1(1, 1, _abi.F32, 1, 1, 7, 1, None, 0, 0, 1, 1, 1, 4, 4, 3, 3,
                                         None) == _abi.ERR_UNSUPPORTED
    assert lib.sfg_hip_kv_gather_pool_v1(1, 1, _abi.F32, 1, 1, 1, 13, 4, 4, 3, 3, 1, 1, None) == _abi.ERR_GUARD


def test_metadata_states_the_lowering_envelope(lib):
    """The metadata string names what the library lowers, as key=value pairs."""
    meta = dict(kv.split("=", 1) for kv in lib.sfg_hip_metadata_v1().decode().split(";")
                if "=" in kv and kv.count("=") == 1)
    assert meta["abi"] == "1" and meta["arch"] == "gfx950"
    assert meta["act"] == "f32,bf16" and meta["head_dim"] == "1..256"
    assert meta["page_tokens"] == "any" and meta["decode_tokens"] == "any"
    assert meta["ffn"] == "dense,moe" and meta["kv"] == "act_dtype"
