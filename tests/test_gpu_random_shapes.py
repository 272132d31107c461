"""Seeded random layer shapes through the GPU layer against the oracle (GPU only).

The hand-picked cases elsewhere follow the BASELINE configurations and the
reference's own test shapes.  Here a fixed generator draws 24 more layers
across the input domain the GPU path accepts, the way the reference's own
decoder accepts them (decoder_compiler.cpp:26-39 validate) -- 24 layers:
  prefill or decode (one to three new tokens per sequence over a paged cache
  of 1..300 tokens, pages of 4, 8 or 16 tokens), dense or MoE (2..8 experts,
  top-1 or top-2), f32 / bf16 / int8 weights, head_dim 4..128, GQA groups
  1..4, ragged sequence lengths and FFN widths.
A second generator draws 12 layers onto the bf16 / int8 MFMA paths, at sizes
where the oracle still takes about a second: prefill of 512..2100 rows in 1..4
ragged sequences at head_dim 64 or 128 (the fused QKV + RoPE epilogue from
1024 rows, the flash kernels), and decode of one or two new tokens for 1..64
sequences over up to 3000 cached tokens in 16-token pages (the MFMA split-KV
kernel and the decode GEMVs), GQA groups 1..16, FFN widths that are and are
not multiples of the GEMM tiles.  A third draws 8 append-mode decode steps
(the step's K / V stored into the pools first, 1..5 new tokens over 1..300
cached ones, pages of 1..32 tokens).
Each layer is checked like the reduced configurations: the output, the
attention output and both residual branches against the oracle (MoE under
the oracle's routing trace, and routed on the device with rows whose oracle
logits are near ties exempt).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from schedforge_amd import CONFIGS

from _helpers import TOL, assert_branches, check_device_routing, decoder_data

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEED = 20261202


def random_configs(n=24, seed=SEED):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        # head_dim 64 / 128 twice as likely: the MFMA flash prefill and decode kernels
        head_dim = int(rng.choice([4, 8, 16, 24, 32, 64, 64, 128, 128]))
        kv_heads = int(rng.choice([1, 2, 4]))
        group = int(rng.choice([1, 2, 4]))
        while kv_heads * group * head_dim > 1024:
            group = max(1, group // 2) if group > 1 else group
            kv_heads = max(1, kv_heads // 2) if group == 1 else kv_heads
        q_heads = kv_heads * group
        moe = bool(rng.random() < 0.5)
        experts = int(rng.choice([2, 4, 8]))
        decode = bool(rng.random() < 0.5)
        kw = dict(hidden=q_heads * head_dim, query_heads=q_heads, kv_heads=kv_heads,
                  head_dim=head_dim, intermediate=int(rng.choice([24, 40, 64, 96, 136, 256])),
                  dtype=str(rng.choice(["f32", "bf16", "w8"])),
                  ffn="moe" if moe else "dense", experts=experts,
                  top_k=int(min(experts, rng.choice([1, 2]))))
        if decode:
            kw.update(batch=int(rng.integers(1, 5)), sequence=int(rng.choice([1, 1, 2, 3])),
                      context_sequence=int(rng.integers(1, 301)),
                      page_tokens=int(rng.choice([4, 8, 16])))
        else:
            kw.update(batch=int(rng.integers(1, 4)), sequence=int(rng.integers(1, 201)),
                      context_sequence=0)
        cfg = CONFIGS["c1"].replace(**kw)
        cfg.validate()
        out.append(cfg)
    return out


def mfma_path_configs(n=12, seed=SEED + 1):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        head_dim = int(rng.choice([64, 128]))
        kv_heads = int(rng.choice([1, 2, 4]))
        group = int(rng.choice([1, 2, 3, 4, 8, 16]))
        while kv_heads * group * head_dim > 2048:
            if group > 1:
                group //= 2
            else:
                kv_heads //= 2
        moe = bool(rng.random() < 0.5)
        experts = int(rng.choice([2, 4, 8, 16]))
        decode = bool(rng.random() < 0.5)
        width = (int(rng.choice([64, 128, 256, 512, 1024, 1408, 2048])) if rng.random() < 0.7
                 else int(8 * rng.integers(8, 257)))
        kw = dict(hidden=kv_heads * group * head_dim, query_heads=kv_heads * group,
                  kv_heads=kv_heads, head_dim=head_dim, intermediate=width,
                  dtype=str(rng.choice(["bf16", "w8"])) if decode else "bf16",
                  ffn="moe" if moe else "dense", experts=experts,
                  top_k=int(min(experts, rng.integers(1, 5))))
        if decode:
            new_tokens = int(rng.choice([1, 1, 1, 1, 2]))
            kw.update(batch=int(rng.integers(1, 65)), sequence=new_tokens,
                      context_sequence=int(rng.integers(new_tokens, 3001)), page_tokens=16)
        else:
            batch = int(rng.integers(1, 5))
            kw.update(batch=batch, sequence=int(rng.integers(max(1, 512 // batch), 2100 // batch + 1)),
                      context_sequence=0)
        cfg = CONFIGS["c1"].replace(**kw)
        cfg.validate()
        out.append(cfg)
    return out


def append_configs(n=8, seed=SEED + 2):
    """Append-mode decode steps (the step's K / V go into the paged pools at
    their true positions first, then the step attends over them): 1..5 new
    tokens over 1..300 cached ones -- more new tokens than cached ones too --
    in pages of 1..32 tokens, with room left in the page tables."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        head_dim = int(rng.choice([4, 12, 32, 64, 80, 128]))
        kv_heads = int(rng.choice([1, 2, 4]))
        group = int(rng.choice([1, 2, 4]))
        moe = bool(rng.random() < 0.5)
        experts = int(rng.choice([2, 4, 8]))
        new_tokens = int(rng.choice([1, 2, 3, 5]))
        context = int(rng.integers(1, 301))
        cfg = CONFIGS["c1"].replace(
            batch=int(rng.integers(1, 9)), sequence=new_tokens, context_sequence=context,
            page_tokens=int(rng.choice([1, 4, 16, 32])), kv_append=True,
            kv_capacity=context + new_tokens + int(rng.integers(0, 40)),
            hidden=kv_heads * group * head_dim, query_heads=kv_heads * group, kv_heads=kv_heads,
            head_dim=head_dim, intermediate=int(8 * rng.integers(2, 65)),
            dtype=str(rng.choice(["f32", "bf16", "w8"])), ffn="moe" if moe else "dense",
            experts=experts, top_k=int(min(experts, rng.choice([1, 2]))))
        cfg.validate()
        out.append(cfg)
    return out


CASES = random_configs()
MFMA_CASES = mfma_path_configs()
APPEND_CASES = append_configs()


def _label(cfg):
    mode = (f"decode{' append' if cfg.kv_append else ''} S{cfg.sequence} "
            f"ctx{cfg.context_sequence} p{cfg.page_tokens}") if cfg.decode \
        else f"prefill B{cfg.batch} S{cfg.sequence}"
    ffn = f"moe E{cfg.experts} k{cfg.top_k}" if cfg.moe else "dense"
    return (f"{mode} {cfg.dtype} H{cfg.hidden} Hq{cfg.query_heads} Hkv{cfg.kv_heads} "
            f"D{cfg.head_dim} I{cfg.intermediate} {ffn}")


def _check_layer(cfg, seed):
    from schedforge_amd.layer import compile_decoder, execute_decoder_layer, layer_taps
    label = _label(cfg)
    print(label, flush=True)
    d = oracle.make_layer_data(cfg, seed)
    ref, rt = oracle.decoder_layer(cfg, d, taps=True)
    # an append plan sizes its page tables for the capacity: identity pages
    perm = None if cfg.kv_append else d.page_permutation
    plan = compile_decoder(cfg, decoder_data(d), "cuda", page_permutation=perm)
    res = execute_decoder_layer(plan, d.input, warmup=0, repetitions=1)
    taps = layer_taps(plan)
    assert np.isfinite(res.output).all(), label
    tol = TOL[cfg.dtype]
    if not cfg.moe:
        assert_branches(d.input, res.output, taps, ref, rt, tol, label)
        return
    differ = check_device_routing(taps, rt, d.router_weight, d.router_bias, cfg.top_k)
    same = np.setdiff1d(np.arange(cfg.rows), differ)
    # row-indexed taps only (an append step's oracle taps also hold the new
    # K / V per sequence)
    sel = lambda t: {k: v[same] for k, v in t.items()
                     if k != "counts" and np.ndim(v) == 2 and len(v) == cfg.rows}
    assert_branches(d.input[same], res.output[same], sel(taps), ref[same], sel(rt), tol,
                    label + ", device routing")
    if cfg.kv_append:
        # an append step advances the plan's cached lengths: the trace run
        # starts again from the same cache in a plan of its own
        d.routing_trace = (rt["ids"], rt["weights"])
        plan = compile_decoder(cfg, decoder_data(d), "cuda", page_permutation=perm)
    else:
        plan.t["trace_ids"] = torch.from_numpy(np.ascontiguousarray(rt["ids"], np.int32)).cuda()
        plan.t["trace_weights"] = torch.from_numpy(np.ascontiguousarray(rt["weights"], np.float32)).cuda()
        plan.desc.use_routing_trace = 1
    res2 = execute_decoder_layer(plan, d.input, warmup=0, repetitions=1)
    assert_branches(d.input, res2.output, layer_taps(plan), ref, rt, tol, label + ", routing trace")


@pytest.mark.parametrize("idx", range(len(CASES)), ids=[f"case{i}" for i in range(len(CASES))])
def test_random_layer_matches_oracle(idx):
    _check_layer(CASES[idx], SEED + idx)


@pytest.mark.parametrize("idx", range(len(MFMA_CASES)),
                         ids=[f"mfma{i}" for i in range(len(MFMA_CASES))])
def test_random_mfma_path_layer_matches_oracle(idx):
    _check_layer(MFMA_CASES[idx], SEED + 200 + idx)


@pytest.mark.parametrize("idx", range(len(APPEND_CASES)),
                         ids=[f"append{i}" for i in range(len(APPEND_CASES))])
def test_random_append_step_matches_oracle(idx):
    _check_layer(APPEND_CASES[idx], SEED + 300 + idx)


@pytest.mark.parametrize("kind", ["prefill f32 D5", "decode bf16 D33", "append w8 D7", "prefill bf16 D1"])
def test_odd_head_dim_layer_matches_oracle(kind):
    """Odd head dims: RoPE rotates the pairs (2i, 2i + 1) and leaves the last
    dimension as it is (apply_rope's loop, decoder_compiler.cpp:101-114), in the
    split kernel (prefill), in the decode attention's Q rotation and in the
    append path's K rotation."""
    base = CONFIGS["c1"].replace(query_heads=6, kv_heads=2, intermediate=200)
    cfg = {
        "prefill f32 D5": base.replace(head_dim=5, hidden=30, batch=2, sequence=37),
        "decode bf16 D33": base.replace(head_dim=33, hidden=198, batch=3, sequence=1, dtype="bf16",
                                        context_sequence=70, page_tokens=8, ffn="moe", experts=4, top_k=2),
        "append w8 D7": base.replace(head_dim=7, hidden=42, batch=2, sequence=3, dtype="w8",
                                     context_sequence=20, page_tokens=4, kv_append=True, kv_capacity=30),
        "prefill bf16 D1": base.replace(head_dim=1, hidden=6, batch=1, sequence=50, dtype="bf16"),
    }[kind]
    _check_layer(cfg, SEED + 400 + len(kind))


def test_append_decode_with_a_qkv_width_the_gemv_tiles_do_not_divide():
    """An append-mode decode step computes the whole QKV product (the new
    tokens' K and V are stored): 32 heads of 4 over one K/V head give a QKV
    width of 136, while every depth (H = I = 128) is one the decode GEMV
    takes.  The plan keeps [N][K] weights -- the fragment-tiled layout needs
    widths the GEMV's column tiles divide -- and the step matches the
    oracle's append mode.  (This shape once planned tiled weights and was
    refused at the QKV product.)"""
    from schedforge_amd import _abi
    from schedforge_amd.layer import compile_decoder, execute_decoder_layer, layer_taps
    cfg = CONFIGS["c2"].replace(batch=2, hidden=128, query_heads=32, kv_heads=1, head_dim=4,
                                intermediate=128, context_sequence=40, kv_append=True,
                                kv_capacity=44)
    d = oracle.make_layer_data(cfg, SEED + 100)
    ref, rt = oracle.decoder_layer(cfg, d, taps=True)
    plan = compile_decoder(cfg, decoder_data(d), "cuda")
    assert plan.layout == _abi.LAYOUT_NK
    res = execute_decoder_layer(plan, d.input, warmup=0, repetitions=1)
    assert_branches(d.input, res.output, layer_taps(plan), ref, rt, TOL[cfg.dtype],
                    "append decode, QKV width 136")
