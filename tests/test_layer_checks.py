"""The layer parity checks themselves, on the CPU: mistakes planted in the
oracle (standing in for a faulty GPU output) must fail them, and the oracle's
own output with the GPU's bf16 roundings must pass.

C2 at its full BASELINE size: a zeroed attention output, a page table that
points a sequence at another sequence's pages (all of them, or a single page)
and an FFN with the wrong silu placement each fail the branch checks at the
bf16 tolerance, although the whole-output error alone stays small for some of
them (the residual stream dominates the output)."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

import oracle
from schedforge_amd import CONFIGS, CONFIG_SEEDS

from _helpers import TOL, assert_branches, branch_errors, check_device_routing, near_tie_rows, route_logits


def _as_gpu_taps(t):
    return {"attn": t["attn_merged"], "residual1": t["residual1"]}


@pytest.fixture(scope="module")
def c2():
    cfg = CONFIGS["c2"]
    d = oracle.make_layer_data(cfg, CONFIG_SEEDS["c2"])
    ref, taps = oracle.decoder_layer(cfg, d, taps=True)
    return cfg, d, ref, taps


def _variant(d, **kw):
    v = SimpleNamespace(**vars(d))
    for k, a in kw.items():
        setattr(v, k, a)
    return v


def test_bf16_rounded_attention_passes(c2):
    """Positive control: round the oracle's attention output to bf16 (what the
    GPU hands the O-projection) and recompute the rest in fp32."""
    cfg, d, ref, taps = c2
    attn = oracle.round_bf16(taps["attn_merged"])
    r1 = (oracle.matmul(attn, d.output_weight) + d.input).astype(np.float32)
    err = branch_errors(d.input, ref - taps["residual1"] + r1, {"attn": attn, "residual1": r1},
                        ref, taps)
    assert max(err.values()) < TOL["bf16"] / 4, err


def test_zeroed_attention_fails(c2):
    cfg, d, ref, taps = c2
    z = _variant(d, cached_value=np.zeros_like(d.cached_value))
    out, t = oracle.decoder_layer(cfg, z, taps=True)
    err = branch_errors(d.input, out, _as_gpu_taps(t), ref, taps)
    print("zeroed attention:", err)
    assert err["attn"] > 0.5 and err["attn_branch"] > 0.5
    with pytest.raises(AssertionError):
        assert_branches(d.input, out, _as_gpu_taps(t), ref, taps, TOL["bf16"])


@pytest.mark.parametrize("pages", [None, 1])
def test_wrong_page_table_fails(c2, pages):
    """A table row pointing at the next sequence's pages: every page (None) or
    only the first 16-token page.  (A permutation of one sequence's own pages is
    invisible by construction: decode attention sums over all cached keys and
    cached K carries no rotation.)"""
    cfg, d, ref, taps = c2
    k, v = d.cached_key.copy(), d.cached_value.copy()
    n = cfg.context_sequence if pages is None else 16 * pages
    k[:, :, :n] = np.roll(d.cached_key, 1, axis=0)[:, :, :n]
    v[:, :, :n] = np.roll(d.cached_value, 1, axis=0)[:, :, :n]
    out, t = oracle.decoder_layer(cfg, _variant(d, cached_key=k, cached_value=v), taps=True)
    err = branch_errors(d.input, out, _as_gpu_taps(t), ref, taps)
    print(f"wrong pages ({pages}):", err)
    with pytest.raises(AssertionError):
        assert_branches(d.input, out, _as_gpu_taps(t), ref, taps, TOL["bf16"])


def test_wrong_ffn_fails(c2):
    """silu on the up projection instead of the gate: only the FFN branch moves."""
    cfg, d, ref, taps = c2
    out, t = oracle.decoder_layer(cfg, _variant(d, gate_weight=d.up_weight, up_weight=d.gate_weight),
                                  taps=True)
    err = branch_errors(d.input, out, _as_gpu_taps(t), ref, taps)
    print("swapped gate/up:", err)
    assert err["attn"] == 0.0 and err["ffn_branch"] > TOL["bf16"]


def test_routing_check_rejects_a_wrong_expert():
    """check_device_routing: a token sent to a different expert without a near
    tie fails (even with a small router-input perturbation); the oracle's own
    routing passes."""
    cfg = CONFIGS["c3"].replace(batch=1, sequence=64, hidden=256, intermediate=128, query_heads=2,
                                kv_heads=1)
    d = oracle.make_layer_data(cfg, 31)
    _, taps = oracle.decoder_layer(cfg, d, taps=True)
    dev = {"route_input": taps["normalized2"], "ids": taps["ids"].copy(), "weights": taps["weights"]}
    assert len(check_device_routing(dev, taps, d.router_weight, d.router_bias, cfg.top_k)) == 0
    logits = route_logits(taps["normalized2"], d.router_weight, d.router_bias)
    ties = set(near_tie_rows(logits, cfg.top_k, 1e-2).tolist())
    row = next(r for r in range(cfg.rows) if r not in ties)
    dev["ids"][row, 0] = next(e for e in range(cfg.experts) if e not in dev["ids"][row])
    with pytest.raises(AssertionError):
        check_device_routing(dev, taps, d.router_weight, d.router_bias, cfg.top_k)
