"""The roofline units bench.py reports (algorithmic_work): FLOPs and bytes
checked against the shapes of the layer's own data and a brute-force count of
the causal mask, not against the formula itself (CPU only)."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from schedforge_amd.configs import algorithmic_work, causal_pairs

from _helpers import SMALL

CASES = [("c1", None), ("c2", None), ("c2", "f32"), ("c3", None), ("c4", None), ("c5", None),
         ("c5", "bf16")]


def _cfg(name, dtype):
    cfg = SMALL[name]
    return cfg if dtype is None else cfg.replace(dtype=dtype)


def _weights(cfg, d):
    """The weights one step reads: a decode step with the reference's
    semantics discards the step's K / V (decoder_compiler.cpp:238-243), so
    only Wq of the QKV weights."""
    qkv = [d.query_weight] if cfg.decode and not cfg.kv_append else [d.query_weight, d.key_weight,
                                                                      d.value_weight]
    ffn = [d.w1, d.w3, d.w2] if cfg.moe else [d.gate_weight, d.up_weight, d.down_weight]
    return qkv + [d.output_weight], ffn


@pytest.mark.parametrize("name,dtype", CASES)
def test_bytes_are_the_bytes_of_the_layer_data(name, dtype):
    cfg = _cfg(name, dtype)
    d = oracle.make_layer_data(cfg, 3)
    w = algorithmic_work(cfg)
    elem = {"f32": 4, "bf16": 2, "w8": 1}[cfg.dtype]
    proj, ffn = _weights(cfg, d)
    router = d.router_weight.size * 4 if cfg.moe else 0   # the router stays fp32
    assert w["weight_bytes"] == sum(a.size for a in proj + ffn) * elem + router
    # the paged pools hold fp32 on the fp32 path, bf16 on the others
    pool = 4 if cfg.dtype == "f32" else 2
    kv = (d.cached_key.size + d.cached_value.size) * pool if cfg.decode else 0
    assert w["kv_bytes"] == kv
    assert w["act_bytes"] == 2 * d.input.nbytes   # fp32 rows in and out
    assert w["bytes"] == w["weight_bytes"] + w["kv_bytes"] + w["act_bytes"]


@pytest.mark.parametrize("name,dtype", CASES)
def test_flops_are_two_per_multiply_add_of_the_layer_products(name, dtype):
    cfg = _cfg(name, dtype)
    d = oracle.make_layer_data(cfg, 3)
    w = algorithmic_work(cfg)
    rows = cfg.rows
    proj, ffn = _weights(cfg, d)
    # a [rows][K] x [K][N] product is rows * K * N multiply-adds
    assert w["proj_flops"] == 2 * rows * sum(a.size for a in proj)
    if cfg.moe:
        per_expert = d.w1[0].size + d.w3[0].size + d.w2[0].size
        expected_ffn = 2 * rows * cfg.top_k * per_expert + 2 * rows * d.router_weight.size
    else:
        expected_ffn = 2 * rows * sum(a.size for a in ffn)
    assert w["ffn_flops"] == expected_ffn
    # attention: QK^T and PV, head_dim multiply-adds each per allowed pair
    skv = cfg.context_sequence if cfg.decode else cfg.sequence
    i = np.arange(cfg.sequence)[:, None]
    j = np.arange(skv)[None, :]
    allowed = int((j <= skv - cfg.sequence + i).sum())
    assert w["attn_flops"] == 2 * 2 * cfg.head_dim * allowed * cfg.batch * cfg.query_heads
    assert w["flops"] == w["proj_flops"] + w["attn_flops"] + w["ffn_flops"]


@pytest.mark.parametrize("sq,skv", [(1, 1), (1, 4096), (2, 2), (5, 9), (7, 7), (3, 40),
                                    (128, 128), (300, 301)])
def test_causal_pairs_count_the_mask(sq, skv):
    """attention_compiler.cpp:68-72: query i sees key j iff j <= Skv - Sq + i."""
    i = np.arange(sq)[:, None]
    j = np.arange(skv)[None, :]
    assert causal_pairs(sq, skv) == int((j <= skv - sq + i).sum())
