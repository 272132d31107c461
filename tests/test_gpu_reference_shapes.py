"""The reference's own test shapes and the generic kernels behind them (GPU only).

The reference tests its decoder layer at H16 D4 (tests/test_schedforge.cpp:
823-893): an fp32 dense prefill (batch 1, seq 4), the same layer with a MoE FFN,
and a decode step over a 16-token cache; its paged-KV test uses head_dim 4,
4-token pages and 7 iota tokens (test_schedforge.cpp:369-409).  None of those
shapes runs on the MFMA kernels (head_dim 64 / 128, 16-token pages, bf16): they
run on the row-per-wave attention kernels, the VALU GEMM and the generic
append / gather kernels.  Each is compared with the oracle on the same seeded
inputs:
  fp32      max|got - ref| / max|ref| below 1e-4 (the north star's fp32 bound),
            and the reference's own max_abs_error < 1e-3 (test:835-837);
  bf16      2e-2; int8 weights 1e-2 against the oracle's int8 path.
Decode steps with more than one new token (S = 2, 3) use the reference's causal
offset: new token i sees cached key j iff j <= context - S + i
(attention_compiler.cpp:68-72).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from schedforge_amd.configs import DecoderConfig

from _helpers import SMALL, TOL, KEEP_ALIVE, assert_branches, check_device_routing, decoder_data, dev

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

# DecoderConfig{1, 4, 16, 32, 4, 2, 4, 1e-5, 1e4, true, Dense, 4, 2} (test_schedforge.cpp:823-825)
REF_DENSE = DecoderConfig(batch=1, sequence=4, hidden=16, intermediate=32, query_heads=4, kv_heads=2,
                          head_dim=4, rms_epsilon=1e-5, rope_theta=1e4, causal=True, ffn="dense",
                          experts=4, top_k=2)
REF_CASES = {
    "dense": REF_DENSE,                                              # test:833-837
    "moe": REF_DENSE.replace(ffn="moe"),                             # test:853-862
    "decode": REF_DENSE.replace(sequence=1, context_sequence=16),    # test:881-893
    "decode-pages4": REF_DENSE.replace(sequence=1, context_sequence=16, page_tokens=4),
    "decode-s2": REF_DENSE.replace(sequence=2, context_sequence=16, page_tokens=4),
    "decode-s3-append": REF_DENSE.replace(sequence=3, context_sequence=13, page_tokens=4,
                                          kv_append=True, kv_capacity=20),
}


def _layer(cfg, seed, trace=False):
    from schedforge_amd.layer import compile_decoder, execute_decoder_layer, layer_taps
    d = oracle.make_layer_data(cfg, seed)
    tr = None
    if trace:
        _, t0 = oracle.decoder_layer(cfg, d, taps=True)
        tr = (t0["ids"], t0["weights"])
        d.routing_trace = tr
    ref, taps = oracle.decoder_layer(cfg, d, taps=True, trace=tr)
    perm = d.page_permutation
    if cfg.kv_append:  # tables sized for the capacity, its pages scattered too
        perm = oracle.page_permutation(seed, cfg.batch * ((cfg.capacity + cfg.page_tokens - 1) // cfg.page_tokens))
    plan = compile_decoder(cfg, decoder_data(d), "cuda", page_permutation=perm)
    res = execute_decoder_layer(plan, d.input, warmup=0, repetitions=1, expected=ref)
    return d, res, layer_taps(plan), ref, taps


@pytest.mark.parametrize("dtype", ["f32", "bf16", "w8"])
@pytest.mark.parametrize("case", list(REF_CASES))
def test_reference_decoder_test_shapes(case, dtype):
    cfg = REF_CASES[case].replace(dtype=dtype)
    seed = 81 + list(REF_CASES).index(case)
    d, res, taps, ref, rt = _layer(cfg, seed)
    assert np.isfinite(res.output).all()
    rows = np.arange(cfg.rows)
    if cfg.moe:
        differ = check_device_routing(taps, rt, d.router_weight, d.router_bias, cfg.top_k)
        rows = np.setdiff1d(rows, differ)
    sel = lambda t: {k: v[rows] for k, v in t.items() if k not in ("counts", "new_k", "new_v")}
    label = f"reference shape {case} {dtype}"
    assert_branches(d.input[rows], res.output[rows], sel(taps), ref[rows], sel(rt), TOL[dtype], label)
    if dtype == "f32":
        # the reference's own acceptance bound for these tests
        assert oracle.max_abs_error(res.output, ref) < 1e-3
    if cfg.moe:
        # the oracle's routing as a trace: every row within tolerance
        d2, res2, taps2, ref2, rt2 = _layer(cfg, seed, trace=True)
        assert_branches(d2.input, res2.output, taps2, ref2, rt2, TOL[dtype], label + " (trace)")


@pytest.mark.parametrize("seq", [2, 5])
@pytest.mark.parametrize("append", [False, True])
def test_decode_with_several_new_tokens_matches_oracle(seq, append):
    """A decode step of S new tokens per sequence at a C2-like shape (head_dim
    128, 16-token pages, bf16): the step's query rows attend under the causal
    offset; in append mode their K / V go into the pools at the true positions
    first and the step attends over them too."""
    cfg = SMALL["c2"].replace(sequence=seq, kv_append=append)
    if append:
        cfg = cfg.replace(kv_capacity=cfg.context_sequence + seq)
    d, res, taps, ref, rt = _layer(cfg, 2000 + 17 * seq + int(append))
    assert_branches(d.input, res.output, taps, ref, rt, TOL["bf16"], f"decode S{seq} append {append}")


# ---------------------------------------------------------------- paged KV
def test_reference_paged_kv_test_on_the_device():
    """test_schedforge.cpp:369-409 on the device: PagedKVConfig{1, 2, 4, 4, 4, 12},
    iota keys / values for 7 tokens; gather returns them in logical order, and
    the paged decode of a 0.125 query (Hq 4, Hkv 2, one row over 7 keys,
    causal) agrees with the contiguous cache (identity table) and with
    reference_attention within 1e-5."""
    from schedforge_amd import kvcache as kv
    keys = np.arange(2 * 7 * 4, dtype=np.float32).reshape(1, 2, 7, 4)
    values = keys + 1.0
    query = np.full((1, 4, 1, 4), 0.125, np.float32)
    outs = []
    for pool in ("f32", "bf16"):
        cache = kv.make_paged_kv_cache(kv.PagedKVConfig(1, 2, 4, 4, 4, 12, pool_dtype=pool))
        kv.append_paged_kv(cache, keys, values, 7)
        assert len(cache.page_table[0]) == 2 and cache.length == 7
        gk, gv = kv.gather_paged_kv(cache)
        np.testing.assert_array_equal(gk, keys)   # iota values <= 56 are exact in bf16 too
        np.testing.assert_array_equal(gv, values)
        outs.append(kv.paged_decode_attention(cache, query, q_heads=4))
    ref = oracle.attention(query, keys, values, causal=True)
    for out in outs:
        assert oracle.max_abs_error(out, ref) < 1e-5
    # the contiguous cache: one sequence's pages in logical order
    flat = kv.make_paged_kv_cache(kv.PagedKVConfig(1, 2, 4, 4, 4, 12, pool_dtype="f32"))
    flat.alloc.free_pages[:] = sorted(flat.alloc.free_pages, reverse=True)  # pops 0, 1, 2
    kv.append_paged_kv(flat, keys, values, 7)
    assert flat.page_table[0] == [0, 1]
    assert oracle.max_abs_error(kv.paged_decode_attention(flat, query, q_heads=4), outs[0]) < 1e-5


def _pools(rng, batch, hkv, lens, d, pt, pps, dtype):
    """fp32 [B][Hkv][L][D] K / V, and the paged pools holding them through a
    random page assignment (K token-major, V token-minor inside a page)."""
    L = max(lens)
    k = rng.standard_normal((batch, hkv, L, d)).astype(np.float32)
    v = rng.standard_normal((batch, hkv, L, d)).astype(np.float32)
    if dtype == "bf16":
        k, v = oracle.round_bf16(k), oracle.round_bf16(v)
    pages = batch * pps
    perm = rng.permutation(pages).astype(np.int32).reshape(batch, pps)
    kp = np.zeros((pages, hkv, pt, d), np.float32)
    vp = np.zeros((pages, hkv, d, pt), np.float32)
    for b in range(batch):
        for t in range(lens[b]):
            pg, sl = perm[b, t // pt], t % pt
            kp[pg, :, sl, :] = k[b, :, t, :]
            vp[pg, :, :, sl] = v[b, :, t, :]
    return k, v, kp, vp, perm


@pytest.mark.parametrize("d,pt,sq,hq,hkv,dtype,splits", [
    (4, 4, 1, 4, 2, "f32", 0), (4, 1, 2, 4, 2, "f32", 3), (8, 4, 3, 6, 2, "f32", 2),
    (16, 32, 1, 8, 1, "bf16", 0), (32, 16, 5, 4, 4, "bf16", 4), (96, 8, 1, 12, 3, "f32", 0),
    (128, 16, 2, 16, 4, "bf16", 0), (128, 16, 1, 32, 1, "bf16", 2), (256, 16, 1, 8, 2, "f32", 0),
    (64, 4, 1, 8, 8, "bf16", 5), (5, 3, 2, 2, 1, "f32", 0), (128, 16, 1, 8, 2, "f32", 0)])
def test_generic_paged_attention_matches_oracle(d, pt, sq, hq, hkv, dtype, splits):
    """sfg_hip_attn_paged_v1 on ragged sequences against reference_attention per
    sequence on the same (for bf16 pools, bf16-rounded) K / V: any head_dim, page
    size, rows per step, GQA ratio (including group 32 and an odd 3), split count
    and pool dtype; fp32 arithmetic throughout, so the fp32 bound holds for
    both pool dtypes."""
    from schedforge_amd import _abi
    lib = _abi.load()
    rng = np.random.default_rng(d * 1000 + pt * 10 + sq)
    batch = 3
    lens = [sq + 7, 3 * pt + sq + 2, 40 + sq][:batch]
    pps = (max(lens) + pt - 1) // pt
    k, v, kp, vp, perm = _pools(rng, batch, hkv, lens, d, pt, pps, dtype)
    q = rng.standard_normal((batch, hq, sq, d)).astype(np.float32)
    if dtype == "bf16":
        kpd, vpd = dev(oracle.to_bf16_bits(kp).view(np.int16)), dev(oracle.to_bf16_bits(vp).view(np.int16))
        kvdt = _abi.BF16
    else:
        kpd, vpd, kvdt = dev(kp), dev(vp), _abi.F32
    qd, tab, lens_d = dev(q), dev(perm), dev(np.asarray(lens, np.int32))
    out = torch.empty((batch, hq, sq, d), dtype=torch.float32, device="cuda")
    KEEP_ALIVE.append(out)
    ws_bytes = lib.sfg_hip_attn_paged_workspace_v1(batch, hq, hkv, sq, d, kvdt, max(lens), pt, splits)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    KEEP_ALIVE.append(ws)
    _abi.check(lib.sfg_hip_attn_paged_v1(
        qd.data_ptr(), kpd.data_ptr(), vpd.data_ptr(), kvdt, tab.data_ptr(), lens_d.data_ptr(),
        out.data_ptr(), _abi.F32, batch, hq, hkv, sq, d, pt, pps, batch * pps, max(lens), 1, splits,
        ctypes.c_float(0.0), 1, ws.data_ptr(), ws.numel(), None))
    got = out.cpu().numpy()
    for b in range(batch):
        ref = oracle.attention(q[b:b + 1], k[b:b + 1, :, :lens[b]], v[b:b + 1, :, :lens[b]], causal=True)
        err = oracle.rel_error(got[b:b + 1], ref)
        assert err < TOL["f32"], (b, err)


# ---------------------------------------------------------------- prefill, GEMM
@pytest.mark.parametrize("d,dtype", [(4, "bf16"), (16, "bf16"), (96, "bf16"), (256, "bf16"),
                                     (5, "f32"), (256, "f32")])
def test_row_prefill_other_head_dims(d, dtype):
    """Prefill at head dims the MFMA kernels do not lower: the row-per-wave
    kernel on bf16 or fp32 operands (fp32 arithmetic), causal and GQA."""
    from schedforge_amd import _abi
    lib = _abi.load()
    rng = np.random.default_rng(d)
    B, hq, hkv, S = 2, 4, 2, 37
    q = rng.standard_normal((B, hq, S, d)).astype(np.float32)
    k = rng.standard_normal((B, hkv, S, d)).astype(np.float32)
    v = rng.standard_normal((B, hkv, S, d)).astype(np.float32)
    if dtype == "bf16":
        q, k, v = oracle.round_bf16(q), oracle.round_bf16(k), oracle.round_bf16(v)
        args = [dev(oracle.to_bf16_bits(a).view(np.int16)) for a in (q, k, v)]
        dt = _abi.BF16
    else:
        args, dt = [dev(a) for a in (q, k, v)], _abi.F32
    out = torch.empty((B, S, hq, d), dtype=torch.float32, device="cuda")
    KEEP_ALIVE.append(out)
    _abi.check(lib.sfg_hip_attn_prefill_v1(args[0].data_ptr(), args[1].data_ptr(), args[2].data_ptr(),
                                           out.data_ptr(), dt, _abi.F32, B, hq, hkv, S, S, d, 1,
                                           ctypes.c_float(0.0), None))
    ref = oracle.attention(q, k, v, causal=True).transpose(0, 2, 1, 3)  # merged [B][S][Hq][D]
    assert oracle.rel_error(out.cpu().numpy(), ref) < TOL["f32"]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("sq,skv,causal,hkv", [(9, 9, True, 2), (5, 7, True, 2), (8, 8, False, 2),
                                               (128, 128, True, 2), (9, 9, True, 1), (3, 11, False, 1)])
def test_reference_attention_test_shapes(sq, skv, causal, hkv, dtype):
    """The shapes of the reference's attention test (test_schedforge.cpp:689-757:
    batch 1, four query heads, head_dim 8; 9 x 9 causal, 5 queries over 7 keys
    with the causal offset j <= Skv - Sq + i, 8 x 8 non-causal, 128 x 128, and
    MQA) through sfg_hip_attn_prefill_v1, against reference_attention on the
    same (for bf16, bf16-rounded) operands."""
    from schedforge_amd import _abi
    lib = _abi.load()
    B, hq, d = 1, 4, 8
    rng = np.random.default_rng(sq * 100 + skv + 7 * hkv + int(causal))
    q = rng.standard_normal((B, hq, sq, d)).astype(np.float32)
    k = rng.standard_normal((B, hkv, skv, d)).astype(np.float32)
    v = rng.standard_normal((B, hkv, skv, d)).astype(np.float32)
    if dtype == "bf16":
        q, k, v = oracle.round_bf16(q), oracle.round_bf16(k), oracle.round_bf16(v)
        args = [dev(oracle.to_bf16_bits(a).view(np.int16)) for a in (q, k, v)]
        dt = _abi.BF16
    else:
        args, dt = [dev(a) for a in (q, k, v)], _abi.F32
    out = torch.empty((B, sq, hq, d), dtype=torch.float32, device="cuda")
    KEEP_ALIVE.append(out)
    _abi.check(lib.sfg_hip_attn_prefill_v1(args[0].data_ptr(), args[1].data_ptr(), args[2].data_ptr(),
                                           out.data_ptr(), dt, _abi.F32, B, hq, hkv, sq, skv, d,
                                           int(causal), ctypes.c_float(0.0), None))
    ref = oracle.attention(q, k, v, causal=causal).transpose(0, 2, 1, 3)  # merged [B][Sq][Hq][D]
    err = oracle.rel_error(out.cpu().numpy(), ref)
    print(f"Sq {sq} Skv {skv} causal {causal} Hkv {hkv} {dtype}: rel err {err:.2e}")
    assert err < TOL["f32"], err


@pytest.mark.parametrize("m,n,k,bdt,epi,grouped", [
    (7, 20, 16, "bf16", 0, False), (33, 24, 48, "bf16", 1, False), (65, 40, 16, "i8", 0, False),
    (70, 24, 16, "bf16", 2, False), (50, 12, 40, "f32", 3, True), (40, 16, 24, "i8", 3, True),
    # sizes that select the larger VALU tiles: 64 x 64 (256+ workgroups) and 32 x 32
    (1024, 1024, 48, "f32", 0, False), (512, 512, 40, "f32", 1, False),
    (1024, 1024, 24, "f32", 2, False), (512, 512, 24, "bf16", 3, False),
    (1024, 256, 40, "i8", 0, True),
    # the reference's int8 matmul test shape, QuantizedMatMulConfig{7, 9, 5}
    # (test_schedforge.cpp:411), without its bias / ReLU (not on the decoder path)
    (7, 9, 5, "i8", 0, False), (7, 9, 5, "i8", 1, False)])
def test_valu_gemm_fallback_is_exact(m, n, k, bdt, epi, grouped):
    """Products the MFMA kernels do not lower (k not a multiple of 32) run on
    the VALU kernel: with small-integer operands every product and partial sum
    is exact in fp32, so the result must equal the fp64 product bit for bit
    (and the SwiGLU / GLU epilogues the fp32 expressions of it); int8 weights
    carry their per-channel scales, grouped problems their row gather.  The
    kernel's tile (64 x 64, 32 x 32, 16 x 32 or 16 x 16, by how many
    workgroups each gives) changes nothing: the shapes cover every one."""
    from schedforge_amd import _abi
    lib = _abi.load()
    rng = np.random.default_rng(m * n + k)
    glu = epi in (2, 3)
    nb = 2 * n if glu else n
    groups = 3 if grouped else 1
    a = rng.integers(-3, 4, (m, k)).astype(np.float32)
    b = rng.integers(-3, 4, (groups, nb, k)).astype(np.float32)
    scales = np.ones((groups, nb), np.float32) if bdt != "i8" else \
        (2.0 ** rng.integers(-3, 2, (groups, nb))).astype(np.float32)
    rows = rng.permutation(m).astype(np.int32) if grouped else None
    offsets = np.array([0, m // 3, m // 3, m], np.int32) if grouped else None  # an empty group too
    resid = rng.integers(-3, 4, (m, n)).astype(np.float32)
    adt = _abi.F32 if bdt == "f32" else _abi.BF16
    ad = dev(a) if adt == _abi.F32 else dev(oracle.to_bf16_bits(a).view(np.int16))
    bd = {"f32": lambda: dev(b), "bf16": lambda: dev(oracle.to_bf16_bits(b).view(np.int16)),
          "i8": lambda: dev(b.astype(np.int8))}[bdt]()
    c = torch.empty((m, n), dtype=torch.float32, device="cuda")
    KEEP_ALIVE.append(c)
    args = _abi.GemmArgs()
    args.a, args.a_dtype, args.lda = ad.data_ptr(), adt, k
    args.b, args.b_dtype, args.ldb = bd.data_ptr(), {"f32": _abi.F32, "bf16": _abi.BF16, "i8": _abi.I8}[bdt], k
    args.b_scales = dev(scales).data_ptr() if bdt == "i8" else None
    args.c, args.c_dtype, args.ldc = c.data_ptr(), _abi.F32, n
    args.residual, args.ldr = dev(resid).data_ptr(), n
    args.m, args.n, args.k, args.epilogue = m, n, k, epi
    args.b_layout, args.tile = _abi.LAYOUT_NK, 0
    if grouped:
        rc = _grouped_gemm(lib, args, dev(rows), dev(offsets), groups, nb * k, nb, m)
    else:
        rc = lib.sfg_hip_gemm_v1(ctypes.byref(args), None, 0, None)
    _abi.check(rc)
    got = c.cpu().numpy()
    ref = np.empty((m, n), np.float64)
    for g in range(groups):
        lo, hi = (offsets[g], offsets[g + 1]) if grouped else (0, m)
        src = a[rows[lo:hi]] if grouped else a[lo:hi]
        prod = (src.astype(np.float64) @ b[g].astype(np.float64).T) * scales[g][None, :]
        if epi == 0:
            ref[lo:hi] = prod
        elif epi == 1:
            ref[lo:hi] = prod + resid[lo:hi]
        else:
            gate, up = prod[:, :n].astype(np.float32), prod[:, n:].astype(np.float32)
            silu = lambda x: x / (1.0 + np.exp(-x.astype(np.float64)))
            ref[lo:hi] = silu(gate) * up if epi == 2 else gate * silu(up)
    if glu:  # silu goes through the device's exp: fp32 tolerance
        assert oracle.rel_error(got, ref) < 1e-5
    else:
        np.testing.assert_array_equal(got, ref.astype(np.float32))


def _grouped_gemm(lib, args, rows, offsets, groups, b_stride, s_stride, limit):
    """The grouped form through the MoE experts entry's GEMM family: a grouped
    problem built in a GemmArgs-compatible call (sfg_hip_gemm_grouped_v1)."""
    return lib.sfg_hip_gemm_grouped_v1(ctypes.byref(args), rows.data_ptr(), limit, offsets.data_ptr(),
                                       groups, b_stride, s_stride, None, 0, None)


@pytest.mark.parametrize("kv_heads", [2, 4])
def test_batch_one_decode_matches_oracle(kv_heads):
    """A decode plan for a single sequence with several KV heads (the MFMA
    split kernel's shape): the pools compile_decoder packs are [page][Hkv][...]
    in memory for a batch of one too."""
    cfg = SMALL["c2"].replace(batch=1, kv_heads=kv_heads)
    d, res, taps, ref, rt = _layer(cfg, 2100 + kv_heads)
    assert_branches(d.input, res.output, taps, ref, rt, TOL["bf16"], f"decode B1 Hkv{kv_heads}")
