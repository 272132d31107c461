"""Whole-layer parity at the full BASELINE sizes of C3, C4 and C5 (GPU only).

The reference checks execute_once against reference_decoder_layer at any shape
(decoder_compiler.cpp:622-673, tests/test_schedforge.cpp:822-900).  Here:
  C3  MoE prefill, 2048 tokens: the whole oracle layer (a few seconds), once
      with routing on the device (rows routed differently must be near ties of
      the oracle's logits) and once under the oracle's own routing trace;
  C4  Llama-3-8B-shaped prefill, S 8192: the whole layer on both sides, every
      row compared (the oracle's register-blocked products take a few tens of
      seconds for it);
  C5  Mixtral-shaped int8 decode, 64 sequences over 8192 cached tokens, every
      row on both sides, routed on the device and under the oracle's trace.
Every check compares the output and, on their own scales, the attention
output and both residual branches (tests/_helpers.py branch_errors).
Tolerances: bf16 2e-2, int8 weights 1e-2 (max|got - ref| / max|ref|).
Exact properties at full size, bit for bit and without the oracle: decode
(C5, C2) under another physical page layout and under reversed batch order,
the MoE prefill (C3) under reversed sequence order, and the causal prefills
(C4, C1) under a changed suffix and with a prefix run as its own sequence.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from schedforge_amd import CONFIGS, CONFIG_SEEDS

from _helpers import TOL, assert_branches, check_device_routing, decoder_data

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _rows(taps, rows):
    return {k: v[rows] for k, v in taps.items() if k != "counts"}


def _compile_and_run(cfg, d, trace=None):
    from schedforge_amd.layer import compile_decoder, execute_decoder_layer, layer_taps
    data = decoder_data(d)
    data.routing_trace = trace
    plan = compile_decoder(cfg, data, "cuda", page_permutation=d.page_permutation)
    res = execute_decoder_layer(plan, d.input, warmup=1, repetitions=1)
    assert np.isfinite(res.output).all()
    return plan, res, layer_taps(plan)


def _rerun(plan, x, trace):
    """The same plan under a routing trace (ids, weights) or, with None, routed
    on the device (decoder_compiler.cpp:281-284)."""
    from schedforge_amd.layer import execute_decoder_layer, layer_taps
    if trace is None:
        plan.t.pop("trace_ids", None)
        plan.t.pop("trace_weights", None)
        plan.desc.use_routing_trace = 0
    else:
        plan.t["trace_ids"] = torch.from_numpy(np.ascontiguousarray(trace[0], np.int32)).cuda()
        plan.t["trace_weights"] = torch.from_numpy(np.ascontiguousarray(trace[1], np.float32)).cuda()
        plan.desc.use_routing_trace = 1
    res = execute_decoder_layer(plan, x, warmup=0, repetitions=1)
    return res, layer_taps(plan)


def test_c3_full_size_matches_oracle():
    cfg = CONFIGS["c3"]
    d = oracle.make_layer_data(cfg, CONFIG_SEEDS["c3"])
    ref, rt = oracle.decoder_layer(cfg, d, taps=True)
    plan, res, taps = _compile_and_run(cfg, d)
    print(f"c3 full: {res.milliseconds:.4f} ms/layer")
    differ = check_device_routing(taps, rt, d.router_weight, d.router_bias, cfg.top_k)
    same = np.setdiff1d(np.arange(cfg.rows), differ)
    assert_branches(d.input[same], res.output[same], _rows(taps, same), ref[same], _rows(rt, same),
                    TOL["bf16"], "c3 full, device routing (rows routed alike)")
    # the oracle's own routing as a trace: every row within tolerance
    res2, taps2 = _rerun(plan, d.input, (rt["ids"], rt["weights"]))
    assert_branches(d.input, res2.output, taps2, ref, rt, TOL["bf16"], "c3 full, routing trace")


def test_c4_full_size_matches_oracle():
    cfg = CONFIGS["c4"]
    d = oracle.make_layer_data(cfg, CONFIG_SEEDS["c4"])
    plan, res, taps = _compile_and_run(cfg, d)
    print(f"c4 full: {res.milliseconds:.4f} ms/layer", flush=True)
    del plan
    torch.cuda.empty_cache()
    ref, rt = oracle.decoder_layer(cfg, d, taps=True)
    assert_branches(d.input, res.output, taps, ref, rt, TOL["bf16"], "c4 full, every row")


def test_c5_full_size_matches_oracle():
    """All 64 decode rows on both sides: routed on the device, then under the
    oracle's own routing as a trace."""
    cfg = CONFIGS["c5"]
    d = oracle.make_layer_data(cfg, CONFIG_SEEDS["c5"])
    plan, res, taps = _compile_and_run(cfg, d)
    print(f"c5 full: {res.milliseconds:.4f} ms/layer")
    quant = oracle.quantize_layer(cfg, d)
    d.w1 = d.w3 = d.w2 = None
    ref, rt = oracle.decoder_layer(cfg, d, quant=quant, taps=True)
    differ = check_device_routing(taps, rt, d.router_weight, d.router_bias, cfg.top_k)
    same = np.setdiff1d(np.arange(cfg.rows), differ)
    assert_branches(d.input[same], res.output[same], _rows(taps, same), ref[same], _rows(rt, same),
                    TOL["w8"], "c5 full, device routing (rows routed alike)")
    res2, taps2 = _rerun(plan, d.input, (rt["ids"], rt["weights"]))
    assert_branches(d.input, res2.output, taps2, ref, rt, TOL["w8"], "c5 full, routing trace")


@pytest.mark.parametrize("name", ["c5", "c2"])
def test_full_size_decode_is_exact_under_page_layout_and_batch_order(name):
    """Two exact properties of a full-size decode step, every stage of which
    works per row or per sequence (attention per sequence over its own pages,
    projections, norms, routing and expert products per row):
      - where the pages sit in the pool does not matter: a second physical
        layout of the same logical caches gives the same bits;
      - reversing the order of the sequences (inputs and their caches)
        reverses the output rows, bit for bit."""
    import copy
    from schedforge_amd.layer import compile_decoder, execute_decoder_layer
    cfg = CONFIGS[name]
    d = oracle.make_layer_data(cfg, CONFIG_SEEDS[name] + 41)

    def run(dd, perm):
        plan = compile_decoder(cfg, decoder_data(dd), "cuda", page_permutation=perm)
        out = execute_decoder_layer(plan, dd.input, warmup=0, repetitions=1).output
        del plan
        torch.cuda.empty_cache()
        return out

    base = run(d, d.page_permutation)
    assert np.isfinite(base).all()
    moved = np.roll(d.page_permutation, 12345)  # same logical pages, other physical slots
    assert not np.array_equal(moved, d.page_permutation)
    assert np.array_equal(run(d, moved), base), "output depends on the physical page layout"
    rev = copy.copy(d)
    rev.input = np.ascontiguousarray(d.input[::-1])
    rev.cached_key = np.ascontiguousarray(d.cached_key[::-1])
    rev.cached_value = np.ascontiguousarray(d.cached_value[::-1])
    assert np.array_equal(run(rev, d.page_permutation), base[::-1]), "batch order changes a row's bits"


def test_c3_full_size_prefill_is_exact_under_batch_order():
    """The full C3 MoE prefill with its four sequences in reverse order gives
    the reversed output, bit for bit: attention stays inside each sequence,
    and every product, norm, routing decision and expert row is computed per
    token whatever the rows an expert tile groups it with."""
    from schedforge_amd.layer import compile_decoder, execute_decoder_layer
    cfg = CONFIGS["c3"]
    d = oracle.make_layer_data(cfg, CONFIG_SEEDS["c3"] + 41)

    def run(x):
        plan = compile_decoder(cfg, decoder_data(d), "cuda", page_permutation=d.page_permutation)
        out = execute_decoder_layer(plan, x, warmup=0, repetitions=1).output
        del plan
        torch.cuda.empty_cache()
        return out

    B, S, H = cfg.batch, cfg.sequence, cfg.hidden
    base = run(d.input)
    assert np.isfinite(base).all()
    rev_in = np.ascontiguousarray(d.input.reshape(B, S, H)[::-1].reshape(B * S, H))
    rev_out = run(rev_in).reshape(B, S, H)[::-1].reshape(B * S, H)
    assert np.array_equal(rev_out, base), "sequence order changes a row's bits"


@pytest.mark.parametrize("name", ["c4", "c1"])
def test_full_size_prefill_is_causal_and_prefix_consistent(name):
    """Two exact properties of the full C4 prefill (one sequence of 8192) and
    of C1's fp32 one (one sequence of 128):
      - causality: changing the second half of the input leaves the first
        half's output bits as they were (masked keys add exact zeros);
      - prefix consistency: the first 4096 rows run as a sequence of their own
        give the same bits as in the full sequence, though the two shapes
        take other GEMM tiles and flash block heights (every such policy
        computes the same arithmetic)."""
    from schedforge_amd.layer import compile_decoder, execute_decoder_layer
    cfg = CONFIGS[name]
    d = oracle.make_layer_data(cfg, CONFIG_SEEDS[name] + 41)
    half = cfg.sequence // 2

    def run(c, x):
        plan = compile_decoder(c, decoder_data(d), "cuda", page_permutation=None)
        out = execute_decoder_layer(plan, x, warmup=0, repetitions=1).output
        del plan
        torch.cuda.empty_cache()
        return out

    base = run(cfg, d.input)
    assert np.isfinite(base).all()
    changed = d.input.copy()
    changed[half:] = changed[half:][::-1] * np.float32(1.5)
    assert np.array_equal(run(cfg, changed)[:half], base[:half]), "a later row changed an earlier output"
    prefix = run(cfg.replace(sequence=half), np.ascontiguousarray(d.input[:half]))
    assert np.array_equal(prefix, base[:half]), "the prefix as its own sequence differs"
