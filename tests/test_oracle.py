"""Pins of the CPU oracle (oracle/sfg_oracle.c) -- CPU only.

Each oracle function is checked against something that does not share its code:
golden vectors written by tests/golden/make_golden.py in float64 NumPy from the
reference's definitions, closed forms, brute force, the reference's own
known-answer tests, and an independent float64 formulation of the whole layer.

  function                 pinned by
  sfgo_rms_norm            golden; closed form x=c -> c w / sqrt(c^2+eps)
  sfgo_matmul              integer operands (exact) vs NumPy int64; bit for bit
                           against the reference's own execute()
                           (tests/test_oracle_ref.py)
  sfgo_rope / split_qkv    golden; position-0 identity; pair norms; known angle
  sfgo_attention           golden (causal + full); equal keys -> prefix mean;
                           one-hot V -> probability row
  sfgo_route_topk          golden ids/weights; ties -> lower index; invariants
                           (test_schedforge.cpp:630-640)
  sfgo_dispatch            golden offsets/tokens/slots (stable argsort)
  sfgo_moe_reference       golden (silu on W3, renormalised weights)
  sfgo_quantize_nk         golden incl. zero column; constant-weight matmul
                           (test_schedforge.cpp:411-417); half-away rounding
  sfgo_quantized_matmul    integer-exact closed form; (x*q)*s rounding order
                           (next_milestones.cpp:60-62) at k = 1, where one fused
                           step is an exact single rounding
  sfgo_quantized_moe       float64 NumPy over dequantized int8 experts (silu on
                           W3, token/slot order); the reference's fp32-MoE bound
                           (test_schedforge.cpp:902-914); int8 MoE layer
  sfgo_to/from_bf16        golden bits incl. ties; test_schedforge.cpp:252-254
  sfgo_paged_gather        iota round trip (test_schedforge.cpp:369-379)
  sfgo_max_abs_error       hand values incl. a NaN (std::max fold, runtime.cpp:628-635)
  sfgo_decoder_layer       float64 NumPy layer (dense prefill, dense decode, MoE,
                           int8 dense, int8 MoE decode)
  sfgo_decoder_layer_rows  bit-exact against the sampled rows (and taps) of
                           sfgo_decoder_layer: dense bf16, MoE with bias and
                           with a trace, int8 dense, two sequences
  generators               determinism, moments, permutation property
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import oracle
from schedforge_amd import CONFIGS

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "golden_v1.npz")


def rel(a, b):
    return oracle.rel_error(a, b)


# ------------------------------------------------------------------ golden vectors
def test_golden_rmsnorm():
    y = oracle.rms_norm(GOLDEN["rms_x"], GOLDEN["rms_w"], 1e-5)
    assert rel(y, GOLDEN["rms_y"]) < 1e-6


@pytest.mark.parametrize("causal,key", [(True, "att_causal"), (False, "att_full")])
def test_golden_attention(causal, key):
    out = oracle.attention(GOLDEN["att_q"], GOLDEN["att_k"], GOLDEN["att_v"], causal)
    assert rel(out, GOLDEN[key]) < 1e-6


def test_golden_route_dispatch_moe():
    ids, w, counts = oracle.route_topk(GOLDEN["route_x"], GOLDEN["route_w"], GOLDEN["route_b"], 2)
    np.testing.assert_array_equal(ids, GOLDEN["route_ids"])
    np.testing.assert_allclose(w, GOLDEN["route_wts"], rtol=1e-6)
    np.testing.assert_array_equal(counts, np.bincount(GOLDEN["route_ids"].reshape(-1), minlength=6))
    c2, off, tok, slots, rw = oracle.dispatch(ids, w, 6)
    np.testing.assert_array_equal(off, GOLDEN["disp_offsets"])
    np.testing.assert_array_equal(tok, GOLDEN["disp_tokens"])
    np.testing.assert_array_equal(slots, GOLDEN["disp_slots"])
    out = oracle.moe_reference(GOLDEN["route_x"], GOLDEN["moe_w1"], GOLDEN["moe_w3"],
                               GOLDEN["moe_w2"], ids, w)
    assert rel(out, GOLDEN["moe_out"]) < 1e-5


def test_golden_quantize():
    q, s = oracle.quantize_kn(GOLDEN["q_w"])
    np.testing.assert_array_equal(q, GOLDEN["q_q"])
    np.testing.assert_array_equal(s, GOLDEN["q_s"])
    assert s[4] == 1.0 and not q[4].any()


def test_golden_rope():
    t = GOLDEN["rope_in"]
    b, h, s, d = t.shape
    qkv = np.zeros((b * s, h * d + 2 * d), np.float32)
    for hh in range(h):
        qkv[:, hh * d:(hh + 1) * d] = t[0, hh]
    q, k, v = oracle.split_qkv_rope(qkv, b, s, h * d, h, 1, d, 10000.0)
    assert rel(q, GOLDEN["rope_out"]) < 1e-6


def test_golden_bf16_bits():
    np.testing.assert_array_equal(oracle.to_bf16_bits(GOLDEN["bf16_in"]), GOLDEN["bf16_bits"])


# ------------------------------------------------------------------ closed forms
def test_rmsnorm_constant_row():
    c, eps = 0.375, 1e-6
    w = np.linspace(0.25, 2.0, 300).astype(np.float32)
    y = oracle.rms_norm(np.full((2, 300), c, np.float32), w, eps)
    np.testing.assert_allclose(y, np.broadcast_to(c * w / np.sqrt(c * c + eps), (2, 300)), rtol=2e-7)


def test_matmul_integer_operands_exact():
    rng = np.random.default_rng(3)
    a = rng.integers(-7, 8, size=(33, 70))
    b = rng.integers(-7, 8, size=(70, 45))
    np.testing.assert_array_equal(oracle.matmul(a.astype(np.float32), b.astype(np.float32)),
                                  (a @ b).astype(np.float32))


def test_rope_identity_at_zero_and_rotation():
    d, s = 8, 3
    rng = np.random.default_rng(5)
    qkv = rng.standard_normal((s, 2 * d + 2 * d)).astype(np.float32)
    q, k, _ = oracle.split_qkv_rope(qkv, 1, s, 2 * d, 2, 1, d, 10000.0)
    np.testing.assert_array_equal(q[0, 0, 0], qkv[0, :d])       # position 0: identity
    # pair norms preserved
    src = qkv[:, :d].reshape(s, d // 2, 2)
    dst = q[0, 0].reshape(s, d // 2, 2)
    np.testing.assert_allclose(np.hypot(*dst.transpose(2, 0, 1)), np.hypot(*src.transpose(2, 0, 1)),
                               rtol=1e-6)
    # pair 0 at position 1 rotates by exactly 1 radian (frequency 1)
    e, o = qkv[1, 0], qkv[1, 1]
    np.testing.assert_allclose(dst[1, 0], [e * np.cos(1.0) - o * np.sin(1.0),
                                           e * np.sin(1.0) + o * np.cos(1.0)], rtol=1e-6)


def test_attention_equal_keys_prefix_mean_and_one_hot():
    rng = np.random.default_rng(7)
    s, d = 9, 8
    q = rng.standard_normal((1, 1, s, d)).astype(np.float32)
    k = np.broadcast_to(rng.standard_normal(d).astype(np.float32), (1, 1, s, d)).copy()
    v = rng.standard_normal((1, 1, s, d)).astype(np.float32)
    out = oracle.attention(q, k, v, True)[0, 0]
    np.testing.assert_allclose(out, np.cumsum(v[0, 0], 0) / np.arange(1, s + 1)[:, None], rtol=1e-5)
    # one-hot values: output row j equals the softmax probability of key j
    k2 = rng.standard_normal((1, 1, s, d)).astype(np.float32)
    eye = np.eye(s, dtype=np.float32)[None, None]
    p = oracle.attention(q, k2, eye, False)[0, 0]
    sc = q[0, 0].astype(np.float64) @ k2[0, 0].T.astype(np.float64) / np.sqrt(d)
    ref = np.exp(sc - sc.max(1, keepdims=True))
    np.testing.assert_allclose(p, ref / ref.sum(1, keepdims=True), rtol=1e-5)


def test_route_ties_and_invariants():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((64, 16)).astype(np.float32)
    r = (rng.standard_normal((16, 5)) * 0.3).astype(np.float32)
    r[:, 3] = r[:, 1]  # experts 1 and 3 always tie: 1 must win
    ids, w, counts = oracle.route_topk(x, r, None, 2)
    assert counts.sum() == 64 * 2                              # test_schedforge.cpp:630-633
    np.testing.assert_allclose(w.sum(1), 1.0, atol=1e-6)        # :634-640
    assert not np.any(ids == 3) or np.all(np.any(ids == 1, 1)[np.any(ids == 3, 1)])
    assert np.all(ids[:, 0] != ids[:, 1])


def test_quantized_constant_matmul():
    """test_schedforge.cpp:411-417: input 0.25, weights 0.2 (7x9, k=5)."""
    w = np.full((5, 9), 0.2, np.float32)
    q, s = oracle.quantize_kn(w)
    assert np.all(q == 127)
    np.testing.assert_allclose(s, np.float32(0.2) / np.float32(127.0))
    y = oracle.quantized_matmul(np.full((7, 5), 0.25, np.float32), q, s)
    assert np.max(np.abs(y - 0.25)) < 0.01


def test_quantize_rounds_half_away_from_zero():
    # column max 127 -> scale 1: values x.5 must round away from zero
    w = np.array([[127.0], [2.5], [-2.5], [0.5], [-0.5], [1.49]], np.float32)
    q, s = oracle.quantize_kn(w)
    assert s[0] == 1.0
    np.testing.assert_array_equal(q[0], [127, 3, -3, 1, -1, 1])


def test_quantized_matmul_integer_exact():
    rng = np.random.default_rng(11)
    q = rng.integers(-127, 128, size=(12, 40)).astype(np.int8)
    s = np.ones(12, np.float32)
    x = rng.integers(-3, 4, size=(5, 40)).astype(np.float32)
    np.testing.assert_array_equal(oracle.quantized_matmul(x, q, s), x @ q.T.astype(np.float32))


def test_quantized_matmul_rounds_x_times_q_first():
    """quantized_invoke forms `acc += x * float(q) * scale` left to right
    (next_milestones.cpp:60-62): x*q rounds to fp32, then one fused
    multiply-add with the scale.  At k = 1 that fused step is a single rounding
    of an exact product, so the expected bits are round32(round32(x*q) * s)
    computed in float64; the other association, x * round32(q*s), differs on
    many of these inputs."""
    rng = np.random.default_rng(12)
    n = 512
    q = rng.integers(-127, 128, size=(n, 1)).astype(np.int8)
    s = (rng.random(n) * 0.01 + 1e-4).astype(np.float32)
    x = rng.standard_normal((64, 1)).astype(np.float32)
    got = oracle.quantized_matmul(x, q, s)
    xq = (x.astype(np.float32) * q.T.astype(np.float32)).astype(np.float32)
    want = (xq.astype(np.float64) * s.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(got, want)
    other = (x * (q.T.astype(np.float32) * s).astype(np.float32)).astype(np.float32)
    assert np.count_nonzero(other != want) > 0


def _np_quantized_moe(x, quant, ids, w):
    """float64 over dequantized experts: gate = x W1, up = silu(x W3),
    out = sum_slot w * ((gate * up) W2) (next_milestones.cpp:418-460)."""
    x = x.astype(np.float64)
    deq = lambda p: (p[0].astype(np.float64) * p[1].astype(np.float64)[:, None]).T   # [K][N]
    out = np.zeros_like(x)
    for t in range(x.shape[0]):
        for sl in range(ids.shape[1]):
            e = ids[t, sl]
            g = x[t] @ deq(quant.e1[e])
            u = x[t] @ deq(quant.e3[e])
            out[t] += w[t, sl] * ((g * (u / (1 + np.exp(-u)))) @ deq(quant.e2[e]))
    return out


def test_quantized_moe_matches_dequantized_float64():
    """sfgo_quantized_moe against float64 NumPy on the dequantized int8
    experts, and against the fp32 MoE on the unquantized weights within the
    reference's own bound (execute_quantized_moe vs its fp32 reference,
    test_schedforge.cpp:902-914: max abs < 0.2)."""
    cfg = CONFIGS["c5"].replace(batch=6, hidden=192, intermediate=160, query_heads=3, kv_heads=1,
                                head_dim=64, context_sequence=32)
    d = oracle.make_layer_data(cfg, 4545)
    quant = oracle.quantize_layer(cfg, d)
    x = oracle.normal(4545, 0, (cfg.batch, cfg.hidden))
    ids, w, _ = oracle.route_topk(x, d.router_weight, None, cfg.top_k)
    got = oracle.quantized_moe(x, quant.e1, quant.e3, quant.e2, ids, w)
    assert rel(got, _np_quantized_moe(x, quant, ids, w)) < 2e-6
    fp32 = oracle.moe_reference(x, d.w1, d.w3, d.w2, ids, w)
    assert np.max(np.abs(got - fp32)) < 0.2
    assert rel(got, fp32) < 2e-2
    # a wrong expert for one slot, or silu on W1 instead of W3, is visible
    bad = ids.copy()
    bad[0, 0] = (bad[0, 0] + 1) % cfg.experts
    if bad[0, 0] == bad[0, 1]:
        bad[0, 0] = (bad[0, 0] + 1) % cfg.experts
    assert rel(oracle.quantized_moe(x, quant.e1, quant.e3, quant.e2, bad, w), got) > 1e-3
    swapped = oracle.quantized_moe(x, quant.e3, quant.e1, quant.e2, ids, w)
    assert rel(swapped, got) > 1e-2


def test_bf16_reference_values():
    vals = np.array([-1.25, 0.0, 0.75, 3.5], np.float32)   # test_schedforge.cpp:252-254
    np.testing.assert_array_equal(oracle.round_bf16(vals), vals)


def test_paged_gather_iota_round_trip():
    """test_schedforge.cpp:369-379 with per-sequence tables: scatter then gather
    reproduces iota keys in logical order."""
    b, h, ctx, d, pt = 2, 2, 7, 4, 4
    keys = np.arange(b * h * ctx * d, dtype=np.float32).reshape(b, h, ctx, d)
    table = np.array([[3, 0], [1, 4]], np.int32)
    pool = oracle.paged_scatter(keys, table, 6, pt)
    np.testing.assert_array_equal(oracle.paged_gather(pool, table, b, h, ctx, pt, d), keys)
    # page 3, kv head 1, token 2 of sequence 0 holds logical token 2
    np.testing.assert_array_equal(pool[3, 1, 2], keys[0, 1, 2])


# ------------------------------------------------------------------ whole layer
def _np_layer(cfg, d, quant=None, appended=None):
    """Independent float64 formulation of reference_decoder_layer; with
    `appended` = (k, v) the build's append mode: the step rotates at its true
    positions and attends over the cache followed by these stored K/V."""
    x = d.input.astype(np.float64)
    B, S, H, Hq, Hkv, D = cfg.batch, cfg.sequence, cfg.hidden, cfg.query_heads, cfg.kv_heads, cfg.head_dim

    def rms(v, w):
        return v / np.sqrt((v ** 2).mean(1, keepdims=True) + cfg.rms_epsilon) * w

    def W(name, i=None):
        if quant is None:
            return getattr(d, name).astype(np.float64)
        q, s = quant.dense[i]
        return (q.astype(np.float64) * s[:, None].astype(np.float64)).T

    n1 = rms(x, d.rms1_weight)
    qkv = np.concatenate([n1 @ W("query_weight", 0), n1 @ W("key_weight", 1), n1 @ W("value_weight", 2)], 1)
    q = qkv[:, :H].reshape(B, S, Hq, D).transpose(0, 2, 1, 3)
    k = qkv[:, H:H + Hkv * D].reshape(B, S, Hkv, D).transpose(0, 2, 1, 3)
    v = qkv[:, H + Hkv * D:].reshape(B, S, Hkv, D).transpose(0, 2, 1, 3)
    pos0 = cfg.context_sequence if appended is not None else 0
    pos = (pos0 + np.arange(S))[:, None].astype(np.float32)
    fr = np.float32(cfg.rope_theta) ** (-np.arange(0, D, 2, dtype=np.float32) / np.float32(D))
    ang = (pos * fr).astype(np.float64)

    def rope(t):
        e, o = t[..., 0::2].copy(), t[..., 1::2].copy()
        t = t.copy()
        t[..., 0::2] = e * np.cos(ang) - o * np.sin(ang)
        t[..., 1::2] = e * np.sin(ang) + o * np.cos(ang)
        return t

    q, k = rope(q), rope(k)
    if appended is not None:
        k = np.concatenate([d.cached_key.astype(np.float64), appended[0].astype(np.float64)], 2)
        v = np.concatenate([d.cached_value.astype(np.float64), appended[1].astype(np.float64)], 2)
    elif cfg.context_sequence > 0:
        k, v = d.cached_key.astype(np.float64), d.cached_value.astype(np.float64)
    skv = k.shape[2]
    g = Hq // Hkv
    k, v = np.repeat(k, g, 1), np.repeat(v, g, 1)
    s = q @ k.transpose(0, 1, 3, 2) / np.sqrt(D)
    if cfg.causal:
        for i in range(S):
            s[:, :, i, skv - S + i + 1:] = -np.inf
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    o = (p @ v).transpose(0, 2, 1, 3).reshape(B * S, H)
    r1 = o @ W("output_weight", 3) + x
    n2 = rms(r1, d.rms2_weight)
    if cfg.ffn == "moe":
        ids, w, _ = oracle.route_topk(n2.astype(np.float32), d.router_weight, d.router_bias, cfg.top_k)
        if quant is not None:
            return r1 + _np_quantized_moe(n2, quant, ids, w)
        f = np.zeros_like(r1)
        for t in range(B * S):
            for sl in range(cfg.top_k):
                e = ids[t, sl]
                gg = n2[t] @ d.w1[e]
                uu = n2[t] @ d.w3[e]
                f[t] += w[t, sl] * ((gg * uu / (1 + np.exp(-uu))) @ d.w2[e])
        return r1 + f
    gate, up = n2 @ W("gate_weight", 4), n2 @ W("up_weight", 5)
    return r1 + (gate / (1 + np.exp(-gate)) * up) @ W("down_weight", 6)


@pytest.mark.parametrize("name,overrides", [
    ("c1", {}),
    ("c2", {"batch": 2, "hidden": 256, "intermediate": 512, "query_heads": 2, "kv_heads": 1,
            "context_sequence": 100}),
    ("c3", {"batch": 1, "sequence": 24, "hidden": 128, "intermediate": 96, "query_heads": 2,
            "kv_heads": 1, "head_dim": 64}),
])
def test_layer_matches_float64_formulation(name, overrides):
    cfg = CONFIGS[name].replace(**overrides)
    d = oracle.make_layer_data(cfg, 4242)
    out = oracle.decoder_layer(cfg, d)
    assert rel(out, _np_layer(cfg, d)) < 2e-6


def test_append_mode_layer_matches_float64_formulation():
    """The build's append mode (not a reference mode): the step's Q and K rotate
    at position `context`, its K/V are stored as bf16 and attended over with the
    cache.  The stored K/V are the fp64 rotation rounded to bf16 (to one bf16
    ulp: fp32 vs fp64 can straddle a rounding boundary), and the layer output
    matches the fp64 formulation that appends exactly those values."""
    cfg = CONFIGS["c2"].replace(batch=2, hidden=256, intermediate=512, query_heads=2, kv_heads=1,
                                context_sequence=100, kv_append=True)
    d = oracle.make_layer_data(cfg, 4243)
    out, taps = oracle.decoder_layer(cfg, d, taps=True)
    new_k, new_v = taps["new_k"], taps["new_v"]
    assert new_k.shape == (2, 1, 1, 128)
    # stored values are bf16
    np.testing.assert_array_equal(oracle.round_bf16(new_k), new_k)
    # K rotated at position 100 (not 0): compare with the unrotated / rotated fp64 projection
    n1 = taps["normalized1"].astype(np.float64)
    kproj = (n1 @ d.key_weight.astype(np.float64)).reshape(2, 1, 1, 128)
    fr = np.float32(cfg.rope_theta) ** (-np.arange(0, 128, 2, dtype=np.float32) / np.float32(128))
    ang = (np.float32(100) * fr).astype(np.float64)
    rot = kproj.copy()
    rot[..., 0::2] = kproj[..., 0::2] * np.cos(ang) - kproj[..., 1::2] * np.sin(ang)
    rot[..., 1::2] = kproj[..., 0::2] * np.sin(ang) + kproj[..., 1::2] * np.cos(ang)
    assert np.max(np.abs(new_k - rot) / np.maximum(np.abs(rot), 1e-3)) < 2 ** -7
    assert np.max(np.abs(new_k - kproj)) > 1e-2  # position 100, not the reference's 0
    vproj = (n1 @ d.value_weight.astype(np.float64)).reshape(2, 1, 1, 128)
    assert np.max(np.abs(new_v - vproj) / np.maximum(np.abs(vproj), 1e-3)) < 2 ** -7
    assert rel(out, _np_layer(cfg, d, appended=(new_k, new_v))) < 2e-6
    # and it is not the reference's decode step
    ref_mode = oracle.decoder_layer(cfg.replace(kv_append=False), d)
    assert rel(out, ref_mode) > 1e-4


def test_int8_dense_layer_matches_dequantized_float64():
    cfg = CONFIGS["c2"].replace(batch=2, hidden=256, intermediate=512, query_heads=2, kv_heads=1,
                                context_sequence=64, dtype="w8")
    d = oracle.make_layer_data(cfg, 4343)
    q = oracle.quantize_layer(cfg, d)
    out = oracle.decoder_layer(cfg, d, quant=q)
    assert rel(out, _np_layer(cfg, d, quant=q)) < 2e-6


def test_int8_moe_layer_matches_dequantized_float64():
    """The C5 path (int8 projections, paged decode over the cache, int8 experts)
    at a reduced shape, against float64 over the dequantized weights."""
    cfg = CONFIGS["c5"].replace(batch=4, hidden=256, intermediate=192, query_heads=4, kv_heads=2,
                                head_dim=64, context_sequence=48)
    d = oracle.make_layer_data(cfg, 4646)
    q = oracle.quantize_layer(cfg, d)
    out = oracle.decoder_layer(cfg, d, quant=q)
    assert rel(out, _np_layer(cfg, d, quant=q)) < 2e-6


def test_routing_trace_replaces_router():
    cfg = CONFIGS["c3"].replace(batch=1, sequence=16, hidden=128, intermediate=64, query_heads=2,
                                kv_heads=1, head_dim=64)
    d = oracle.make_layer_data(cfg, 77)
    out, taps = oracle.decoder_layer(cfg, d, taps=True)
    out2 = oracle.decoder_layer(cfg, d, trace=(taps["ids"], taps["weights"]))
    np.testing.assert_array_equal(out, out2)


@pytest.mark.parametrize("name,overrides,trace", [
    ("c4", {"batch": 2, "sequence": 96, "hidden": 256, "intermediate": 384, "query_heads": 2,
            "kv_heads": 1}, False),
    ("c3", {"batch": 2, "sequence": 64, "hidden": 256, "intermediate": 128, "query_heads": 2,
            "kv_heads": 1}, False),
    ("c3", {"batch": 1, "sequence": 80, "hidden": 256, "intermediate": 128, "query_heads": 2,
            "kv_heads": 1}, True),
    ("c4", {"batch": 1, "sequence": 64, "hidden": 256, "intermediate": 256, "query_heads": 2,
            "kv_heads": 1, "dtype": "w8"}, False),
    ("c1", {}, False),
])
def test_row_sampled_layer_equals_full_layer_rows(name, overrides, trace):
    """sfgo_decoder_layer_rows (the full-size C4 checker) is the full layer at
    the sampled rows, bit for bit, taps included."""
    cfg = CONFIGS[name].replace(**overrides)
    d = oracle.make_layer_data(cfg, 5151)
    q = oracle.quantize_layer(cfg, d) if cfg.dtype == "w8" else None
    tr = None
    if trace:
        _, t0 = oracle.decoder_layer(cfg, d, taps=True)
        tr = (t0["ids"], t0["weights"])
    full, taps = oracle.decoder_layer(cfg, d, quant=q, taps=True, trace=tr)
    rows = cfg.batch * cfg.sequence
    sample = np.unique(np.r_[0, 1, cfg.sequence - 1, rows - 1, np.arange(3, rows, 7)])
    got, gt = oracle.decoder_layer_rows(cfg, d, sample, quant=q, taps=True, trace=tr)
    np.testing.assert_array_equal(got, full[sample])
    for key in ("normalized1", "qkv", "attn_merged", "residual1", "normalized2"):
        np.testing.assert_array_equal(gt[key], taps[key][sample], err_msg=key)
    if cfg.ffn == "moe":
        np.testing.assert_array_equal(gt["ids"], taps["ids"][sample])
        np.testing.assert_array_equal(gt["weights"], taps["weights"][sample])


# ------------------------------------------------------------------ generators
def test_generator_determinism_and_moments():
    a = oracle.normal(1000, "wq", (4096,), 0.02)
    b = oracle.normal(1000, "wq", (4096,), 0.02)
    c = oracle.normal(1000, "wk", (4096,), 0.02)
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(a, c)
    big = oracle.normal(7, 0, (200000,))
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1.0) < 0.01
    perm = oracle.page_permutation(5, 1000)
    np.testing.assert_array_equal(np.sort(perm), np.arange(1000))
    assert not np.array_equal(perm, np.arange(1000))


def test_oracle_rejects_invalid_config():
    cfg = CONFIGS["c1"].replace(hidden=250)  # hidden != Hq * D
    d = oracle.make_layer_data(CONFIGS["c1"], 1)
    with pytest.raises(ValueError):
        oracle.decoder_layer(cfg, d)
