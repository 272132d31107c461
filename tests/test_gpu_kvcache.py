"""Paged KV cache on the device (GPU only): append / gather / truncate / release
(next_milestones.cpp:472-581) through libsfg_hip.so, decode attention over an
appended cache, and the decoder layer's append mode (true-position RoPE, the
step's K/V written into the pools) step by step against the oracle.

Append and gather move bf16 bits: exact.  Attention and layer outputs: 2e-2
relative (bf16)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
from schedforge_amd import CONFIG_SEEDS, _abi
from schedforge_amd.kvcache import (PagedKVConfig, append_paged_kv, gather_paged_kv, gather_plan_kv,
                                    make_paged_kv_cache, release_paged_kv_pages, truncate_paged_kv)

from _helpers import SMALL, TOL, decoder_data, dev

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def test_append_gather_iota_round_trip():
    """test_schedforge.cpp:369-390 at head_dim 128 / 16-token pages: iota
    values (exact in bf16) appended over two pages come back in logical order;
    an active page cannot be released; truncation frees the tail page."""
    cfg = PagedKVConfig(1, 2, 128, 128, 16, 48)
    cache = make_paged_kv_cache(cfg)
    n = 2 * 23 * 128
    keys = (np.arange(n) % 256 - 128).astype(np.float32).reshape(1, 2, 23, 128)
    values = keys + 1.0
    append_paged_kv(cache, keys, values, 23)
    assert len(cache.page_table[0]) == 2 and cache.length == 23
    k, v = gather_paged_kv(cache)
    np.testing.assert_array_equal(k, keys)
    np.testing.assert_array_equal(v, values)
    with pytest.raises(ValueError, match="active"):
        release_paged_kv_pages(cache, [cache.page_table[0][0]])
    pages = len(cache.page_table[0])
    truncate_paged_kv(cache, 3)
    assert cache.length == 3 and len(cache.page_table[0]) < pages and cache.free_pages
    k3, _ = gather_paged_kv(cache)
    np.testing.assert_array_equal(k3, keys[:, :, :3])
    with pytest.raises(ValueError, match="capacity"):
        append_paged_kv(cache, np.zeros((1, 2, 46, 128), np.float32),
                        np.zeros((1, 2, 46, 128), np.float32), 46)


def test_append_in_chunks_across_pages_and_sequences():
    cfg = PagedKVConfig(3, 2, 128, 128, 16, 80)
    cache = make_paged_kv_cache(cfg)
    chunks = [10, 13, 20, 1]
    ks, vs = [], []
    for i, t in enumerate(chunks):
        k = oracle.round_bf16(oracle.normal(301, 2 * i, (3, 2, t, 128)))
        v = oracle.round_bf16(oracle.normal(301, 2 * i + 1, (3, 2, t, 128)))
        bits = i % 2 == 1  # alternate fp32 and bf16-bit sources
        append_paged_kv(cache, dev(oracle.to_bf16_bits(k).view(np.int16)) if bits else k,
                        dev(oracle.to_bf16_bits(v).view(np.int16)) if bits else v, t)
        ks.append(k)
        vs.append(v)
    k, v = gather_paged_kv(cache)
    np.testing.assert_array_equal(k, np.concatenate(ks, 2))
    np.testing.assert_array_equal(v, np.concatenate(vs, 2))
    assert len({p for t in cache.page_table for p in t}) == 3 * 3


def test_paged_decode_over_appended_cache_matches_contiguous():
    """The reference's invariant (test_schedforge.cpp:392-409): decode attention
    walking the pages of an appended cache equals attention over the gathered
    contiguous K/V."""
    B, Hq, Hkv, D, T = 2, 8, 2, 128, 37
    cache = make_paged_kv_cache(PagedKVConfig(B, Hkv, D, D, 16, 64))
    k = oracle.round_bf16(oracle.normal(302, 0, (B, Hkv, T, D)))
    v = oracle.round_bf16(oracle.normal(302, 1, (B, Hkv, T, D)))
    append_paged_kv(cache, k, v, T)
    q = oracle.normal(302, 2, (B, Hq, 1, D))
    lib = _abi.load()
    c = cache.config
    ws = torch.empty(lib.sfg_hip_attn_decode_workspace_v1(B, Hq, D, T, 16, 0), dtype=torch.uint8,
                     device="cuda")
    out = torch.empty((B, Hq * D), dtype=torch.float32, device="cuda")
    _abi.check(lib.sfg_hip_attn_decode_paged_v1(
        dev(q).data_ptr(), cache.k_pool.data_ptr(), cache.v_pool.data_ptr(), cache.table.data_ptr(),
        None, out.data_ptr(), _abi.F32, B, Hq, Hkv, D, 16, c.pages_per_seq, c.num_pages, T, 0,
        ctypes.c_float(0.0), 1, ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    ref = oracle.attention(oracle.round_bf16(q), k, v, True).reshape(B, Hq * D)
    assert oracle.rel_error(out.cpu().numpy(), ref) < 2e-2


def test_layer_append_mode_steps_match_oracle():
    """Three decode steps of a plan in append mode: each step's output, and the
    K/V it appended, against the oracle's append mode over the cache as the
    device holds it before the step; lengths advance on the device; a step past
    the page tables' capacity is refused on the host."""
    from schedforge_amd.layer import compile_decoder, run_layer
    base = SMALL["c2"]
    ctx = base.context_sequence
    cfg = base.replace(kv_append=True, kv_capacity=ctx + 3)
    d = oracle.make_layer_data(cfg, CONFIG_SEEDS["c2"] + 7)
    plan = compile_decoder(cfg, decoder_data(d), "cuda")
    assert plan.desc.kv_append == 1 and plan.desc.pages_per_seq * 16 >= ctx + 3
    x = torch.from_numpy(d.input).cuda()
    out = torch.empty((cfg.rows, cfg.hidden), dtype=torch.float32, device="cuda")
    for step in range(3):
        length = ctx + step
        k_cache, v_cache = gather_plan_kv(plan, length)
        d.cached_key, d.cached_value = k_cache, v_cache
        ref, taps = oracle.decoder_layer(cfg.replace(context_sequence=length), d, taps=True)
        run_layer(plan, x, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        err = oracle.rel_error(got, ref)
        print(f"append step {step} (length {length}): rel_err {err:.3e}")
        assert np.isfinite(got).all() and err < TOL[cfg.dtype], err
        k_all, v_all = gather_plan_kv(plan, length + 1)
        np.testing.assert_array_equal(k_all[:, :, :length], k_cache)   # cache untouched
        assert oracle.rel_error(k_all[:, :, length:], taps["new_k"]) < 2e-2
        assert oracle.rel_error(v_all[:, :, length:], taps["new_v"]) < 2e-2
    assert (plan.t["seq_lens"].cpu().numpy() == ctx + 3).all()
    with pytest.raises(ValueError, match="capacity"):
        run_layer(plan, x, out)


def test_append_at_capacity_writes_nothing_and_lengths_saturate():
    """Device guard at the capacity boundary (the host mirror refuses the step,
    as append_paged_kv does, next_milestones.cpp:498): a sequence already at
    pages_per_seq * 16 tokens gets no K/V written and keeps its length; one
    token short appends its last token and reaches the capacity."""
    lib = _abi.load()
    B, Hkv, D, PT, pps = 2, 2, 128, 16, 2
    cap = pps * PT
    pages = B * pps
    table = np.arange(pages, dtype=np.int32).reshape(B, pps)
    k_pool = torch.zeros((pages, Hkv, PT, D), dtype=torch.int16, device="cuda")
    v_pool = torch.zeros((pages, Hkv, D, PT), dtype=torch.int16, device="cuda")
    lens = dev(np.array([cap, cap - 1], np.int32))
    keys = np.full((B, Hkv, 1, D), 3.0, np.float32)
    _abi.check(lib.sfg_hip_kv_append_paged_v1(
        dev(keys).data_ptr(), dev(keys + 1).data_ptr(), _abi.F32, k_pool.data_ptr(),
        v_pool.data_ptr(), dev(table).data_ptr(), lens.data_ptr(), 0, 1, B, Hkv, 1, D, PT, pps,
        pages, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(lens.cpu().numpy(), [cap, cap])
    kp = k_pool.cpu().numpy()
    # sequence 0 (full): untouched; sequence 1: its last slot holds bf16(3.0) = 0x4040
    assert not kp[table[0]].any()
    assert (kp[table[1, 1], :, PT - 1].view(np.uint16) == 0x4040).all()
    assert not kp[table[1, 1], :, :PT - 1].any() and not kp[table[1, 0]].any()
