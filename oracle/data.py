"""Seeded decoder-layer inputs and the whole-layer oracle call (test infrastructure).

make_layer_data(cfg, seed) draws every tensor from the counter-based generator
(tensor ids in oracle.TID): activations N(0,1), weights N(0,0.02), norm gains 1,
cached K/V N(0,1), router bias N(0, cfg.router_bias_std) when that is > 0.
bf16 configs round activations, weights and the KV cache to bf16 (RNE);
w8 configs round activations and the KV cache, and quantize projection and
expert weights per output channel (quantize_layer).
"""
from __future__ import annotations

import ctypes
from types import SimpleNamespace

import numpy as np

from . import (LayerCfg, LayerData, LayerTaps, _b, _f, _i, lib, normal, page_permutation,
               quantize_kn, round_bf16)

WEIGHT_STD = 0.02


def make_layer_data(cfg, seed: int) -> SimpleNamespace:
    H, I, D = cfg.hidden, cfg.intermediate, cfg.head_dim
    kvd = cfg.kv_heads * D
    rows = cfg.batch * cfg.sequence
    d = SimpleNamespace()
    d.input = normal(seed, "x", (rows, H))
    d.rms1_weight = np.ones(H, np.float32)
    d.rms2_weight = np.ones(H, np.float32)
    d.query_weight = normal(seed, "wq", (H, H), WEIGHT_STD)
    d.key_weight = normal(seed, "wk", (H, kvd), WEIGHT_STD)
    d.value_weight = normal(seed, "wv", (H, kvd), WEIGHT_STD)
    d.output_weight = normal(seed, "wo", (H, H), WEIGHT_STD)
    d.gate_weight = d.up_weight = d.down_weight = None
    d.router_weight = d.router_bias = d.w1 = d.w3 = d.w2 = None
    if cfg.ffn == "moe":
        E = cfg.experts
        d.router_weight = normal(seed, "router", (H, E), WEIGHT_STD)
        if getattr(cfg, "router_bias_std", 0.0) > 0.0:
            d.router_bias = normal(seed, "router_bias", (E,), cfg.router_bias_std)
        d.w1 = normal(seed, "w1", (E, H, I), WEIGHT_STD)
        d.w3 = normal(seed, "w3", (E, H, I), WEIGHT_STD)
        d.w2 = normal(seed, "w2", (E, I, H), WEIGHT_STD)
    else:
        d.gate_weight = normal(seed, "wg", (H, I), WEIGHT_STD)
        d.up_weight = normal(seed, "wu", (H, I), WEIGHT_STD)
        d.down_weight = normal(seed, "wd", (I, H), WEIGHT_STD)
    d.cached_key = d.cached_value = None
    d.page_permutation = None
    if cfg.context_sequence > 0:
        ctx = cfg.context_sequence
        d.cached_key = normal(seed, "k_cache", (cfg.batch, cfg.kv_heads, ctx, D))
        d.cached_value = normal(seed, "v_cache", (cfg.batch, cfg.kv_heads, ctx, D))
        pps = (ctx + cfg.page_tokens - 1) // cfg.page_tokens
        d.page_permutation = page_permutation(seed, cfg.batch * pps)
    d.routing_trace = None
    if cfg.dtype in ("bf16", "w8"):
        d.input = round_bf16(d.input)
        if d.cached_key is not None:
            d.cached_key = round_bf16(d.cached_key)
            d.cached_value = round_bf16(d.cached_value)
    if cfg.dtype == "bf16":
        for name in ("query_weight", "key_weight", "value_weight", "output_weight", "gate_weight",
                     "up_weight", "down_weight", "router_weight", "w1", "w3", "w2"):
            v = getattr(d, name)
            if v is not None:
                setattr(d, name, round_bf16(v))
    return d


def quantize_layer(cfg, d) -> SimpleNamespace:
    """Per-channel int8 of every projection / FFN weight (quantize_decoder_weights,
    next_milestones.cpp:660-674; quantize_moe_weights, 699-714)."""
    q = SimpleNamespace()
    names = ["query_weight", "key_weight", "value_weight", "output_weight"]
    if cfg.ffn != "moe":
        names += ["gate_weight", "up_weight", "down_weight"]
    q.dense = [quantize_kn(getattr(d, n)) for n in names]
    if cfg.ffn == "moe":
        E = cfg.experts
        q.e1 = [quantize_kn(d.w1[e]) for e in range(E)]
        q.e3 = [quantize_kn(d.w3[e]) for e in range(E)]
        q.e2 = [quantize_kn(d.w2[e]) for e in range(E)]
    return q


def _stack(pairs):
    qs = np.ascontiguousarray(np.stack([p[0] for p in pairs]))
    ss = np.ascontiguousarray(np.stack([p[1] for p in pairs]))
    return qs, ss


def _layer_structs(cfg, d, quant, threads, trace):
    """LayerCfg / LayerData for one call, plus the arrays they point into."""
    c = LayerCfg(cfg.batch, cfg.sequence, cfg.hidden, cfg.intermediate, cfg.query_heads,
                 cfg.kv_heads, cfg.head_dim, cfg.rms_epsilon, cfg.rope_theta, int(cfg.causal),
                 int(cfg.ffn == "moe"), cfg.experts, cfg.top_k, cfg.context_sequence,
                 int(cfg.dtype == "w8"), threads, int(getattr(cfg, "kv_append", False)),
                 int(cfg.dtype == "f32"))
    ld = LayerData()
    keep = []

    def F(a):
        if a is None:
            return None
        a = np.ascontiguousarray(a, np.float32)
        keep.append(a)
        return _f(a)

    ld.input, ld.rms1, ld.rms2 = F(d.input), F(d.rms1_weight), F(d.rms2_weight)
    ld.wq, ld.wk, ld.wv, ld.wo = F(d.query_weight), F(d.key_weight), F(d.value_weight), F(d.output_weight)
    ld.wg, ld.wu, ld.wd = F(d.gate_weight), F(d.up_weight), F(d.down_weight)
    ld.router, ld.router_bias = F(d.router_weight), F(d.router_bias)
    if cfg.dtype != "w8":
        ld.w1, ld.w3, ld.w2 = F(d.w1), F(d.w3), F(d.w2)
    ld.cached_k, ld.cached_v = F(d.cached_key), F(d.cached_value)
    if trace is not None:
        ids = np.ascontiguousarray(trace[0], np.int32)
        wts = np.ascontiguousarray(trace[1], np.float32)
        keep += [ids, wts]
        ld.trace_ids, ld.trace_weights = _i(ids), _f(wts)
    if cfg.dtype == "w8":
        if quant is None:
            quant = quantize_layer(cfg, d)
        for j, (qq, ss) in enumerate(quant.dense):
            keep += [qq, ss]
            ld.q8[j] = _b(qq)
            ld.s8[j] = _f(ss)
        if cfg.ffn == "moe":
            for name, pairs in (("e1", quant.e1), ("e3", quant.e3), ("e2", quant.e2)):
                qs, ss = _stack(pairs)
                keep += [qs, ss]
                setattr(ld, name + "q", _b(qs))
                setattr(ld, name + "s", _f(ss))
    return c, ld, keep


def _taps(cfg, rows):
    H = cfg.hidden
    kvd = cfg.kv_heads * cfg.head_dim
    t = {"normalized1": np.empty((rows, H), np.float32),
         "qkv": np.empty((rows, H + 2 * kvd), np.float32),
         "attn_merged": np.empty((rows, H), np.float32),
         "residual1": np.empty((rows, H), np.float32),
         "normalized2": np.empty((rows, H), np.float32)}
    tp = LayerTaps(_f(t["normalized1"]), _f(t["qkv"]), _f(t["attn_merged"]),
                   _f(t["residual1"]), _f(t["normalized2"]))
    if getattr(cfg, "kv_append", False):
        t["new_k"] = np.empty((cfg.batch, cfg.kv_heads, cfg.sequence, cfg.head_dim), np.float32)
        t["new_v"] = np.empty_like(t["new_k"])
        tp.new_k, tp.new_v = _f(t["new_k"]), _f(t["new_v"])
    if cfg.ffn == "moe":
        t["ids"] = np.empty((rows, cfg.top_k), np.int32)
        t["weights"] = np.empty((rows, cfg.top_k), np.float32)
        t["counts"] = np.empty(cfg.experts, np.int32)
        tp.ids, tp.weights, tp.counts = _i(t["ids"]), _f(t["weights"]), _i(t["counts"])
    return t, tp


def decoder_layer(cfg, d, quant=None, taps: bool = False, threads: int = 0,
                  trace=None):
    """reference_decoder_layer (decoder_compiler.cpp:622-673) restated; int8 mode
    per next_milestones.cpp.  Returns out [rows, H] (and a dict of taps)."""
    rows = cfg.batch * cfg.sequence
    c, ld, keep = _layer_structs(cfg, d, quant, threads, trace)
    out = np.empty((rows, cfg.hidden), np.float32)
    t, tp = _taps(cfg, rows) if taps else ({}, None)
    rc = lib().sfgo_decoder_layer(ctypes.byref(c), ctypes.byref(ld), _f(out),
                                  ctypes.byref(tp) if tp is not None else None)
    del keep
    if rc != 0:
        raise ValueError("invalid decoder configuration")
    return (out, t) if taps else out


def prepared_layer(cfg, d, quant=None, threads: int = 0):
    """The whole layer as a callable over inputs marshalled once: returns
    run() -> out [rows, H], each call one sfgo_decoder_layer step on the same
    prepared structs (for timing the step itself, without re-stacking the
    expert matrices on every call)."""
    rows = cfg.batch * cfg.sequence
    c, ld, keep = _layer_structs(cfg, d, quant, threads, None)
    out = np.empty((rows, cfg.hidden), np.float32)

    def run():
        rc = lib().sfgo_decoder_layer(ctypes.byref(c), ctypes.byref(ld), _f(out), None)
        if rc != 0:
            raise ValueError("invalid decoder configuration")
        return out

    run.keep = keep  # the arrays the structs point into live as long as run
    return run


def decoder_layer_rows(cfg, d, sample, quant=None, taps: bool = False, threads: int = 0,
                       trace=None):
    """The prefill layer at rows `sample` only (row = b * S + s): K / V of every
    row, everything else for the sampled rows (sfgo_decoder_layer_rows).  Equal
    bit for bit to those rows of decoder_layer.  Returns out [n, H] (and n-row
    taps; "counts" covers the sampled rows)."""
    sample = np.ascontiguousarray(sample, np.int64)
    n = sample.size
    c, ld, keep = _layer_structs(cfg, d, quant, threads, trace)
    out = np.empty((n, cfg.hidden), np.float32)
    t, tp = _taps(cfg, n) if taps else ({}, None)
    rc = lib().sfgo_decoder_layer_rows(ctypes.byref(c), ctypes.byref(ld),
                                       sample.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                       ctypes.c_int64(n), _f(out),
                                       ctypes.byref(tp) if tp is not None else None)
    del keep
    if rc != 0:
        raise ValueError("invalid row-sampled decoder configuration")
    return (out, t) if taps else out
