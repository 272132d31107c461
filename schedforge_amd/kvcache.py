"""Paged KV cache on the device: the reference's PagedKVCache API
(include/schedforge/next_milestones.h:15-43; src/next_milestones.cpp:472-581)
over the gfx950 pools written and read by libsfg_hip.so.

Layout differences, by design (the decode kernels stream one 4 KB run per
(page, kv_head)):
  * one page table per sequence, [B][pages_per_seq], instead of one table
    shared by the batch (the reference's storage is [page][B][Hkv][tok][D]);
  * K pool [page][Hkv][page_tokens][D] and V pool [page][Hkv][D][page_tokens],
    bf16 by default or fp32 (PagedKVConfig.pool_dtype, a build extension: the
    reference stores fp32, so an fp32 pool holds its values exactly).
Pages come from one free list shared by all sequences, initialised 0..N-1 and
popped from the back, as make_paged_kv_cache / append_paged_kv do
(next_milestones.cpp:472-484, 496-501); every guard raises the reference's error
class (ValueError for std::invalid_argument, RuntimeError for std::runtime_error).

PageAllocator is the host bookkeeping alone (no device); PagedKVCache owns the
device pools and moves data only through the HIP kernels (a GPU is required).
"""
from __future__ import annotations

import dataclasses
from typing import List

import numpy as np

from . import _abi
from ._abi import BF16, F32, check


@dataclasses.dataclass
class PagedKVConfig:
    """PagedKVConfig (next_milestones.h:15-22)."""
    batch: int = 1
    kv_heads: int = 1
    head_dim: int = 1
    head_dim_value: int = 1
    page_tokens: int = 16
    capacity: int = 0
    pool_dtype: str = "bf16"    # build extension: "bf16" or "f32"

    def validate(self) -> None:
        """validate_paged_config (next_milestones.cpp:23-27)."""
        if (self.batch <= 0 or self.kv_heads <= 0 or self.head_dim <= 0 or self.head_dim_value <= 0
                or self.page_tokens <= 0 or self.capacity <= 0):
            raise ValueError("invalid paged KV configuration")
        if self.pool_dtype not in ("bf16", "f32"):
            raise ValueError(f"unknown paged KV pool dtype {self.pool_dtype}")

    @property
    def pages_per_seq(self) -> int:
        return (self.capacity + self.page_tokens - 1) // self.page_tokens

    @property
    def num_pages(self) -> int:
        return self.batch * self.pages_per_seq


class PageAllocator:
    """Host page bookkeeping of a paged cache: per-sequence logical -> physical
    page lists, one free list, the cache length, and the reference's guards."""

    def __init__(self, config: PagedKVConfig):
        config.validate()
        self.config = config
        self.length = 0
        self.page_table: List[List[int]] = [[] for _ in range(config.batch)]
        self.free_pages: List[int] = list(range(config.num_pages))

    def reserve(self, tokens: int) -> None:
        """The allocation half of append_paged_kv (next_milestones.cpp:486-501):
        capacity guard, then pages from the back of the free list until every
        sequence's table covers length + tokens."""
        c = self.config
        if tokens <= 0 or self.length + tokens > c.capacity:
            raise ValueError("paged KV capacity exceeded")
        last_page = (self.length + tokens - 1) // c.page_tokens
        for table in self.page_table:
            while len(table) <= last_page:
                if not self.free_pages:
                    raise RuntimeError("paged KV page allocator exhausted")
                table.append(self.free_pages.pop())

    def truncate(self, new_length: int) -> None:
        """truncate_paged_kv (next_milestones.cpp:542-552): tail pages go back to
        the free list."""
        if new_length < 0 or new_length > self.length:
            raise ValueError("invalid paged KV truncation length")
        pt = self.config.page_tokens
        retained = 0 if new_length == 0 else (new_length + pt - 1) // pt
        for table in self.page_table:
            while len(table) > retained:
                self.free_pages.append(table.pop())
        self.length = new_length

    def release(self, pages) -> None:
        """release_paged_kv_pages (next_milestones.cpp:527-540)."""
        for page in pages:
            if page < 0 or page >= self.config.num_pages:
                raise ValueError("invalid physical KV page")
            if any(page in table for table in self.page_table):
                raise ValueError("cannot release an active paged KV page")
            if page not in self.free_pages:
                self.free_pages.append(page)

    def table_array(self) -> np.ndarray:
        """[B][pages_per_seq] int32; unassigned entries are -1 (the kernels skip them)."""
        out = np.full((self.config.batch, self.config.pages_per_seq), -1, dtype=np.int32)
        for b, table in enumerate(self.page_table):
            out[b, :len(table)] = table
        return out


class PagedKVCache:
    """PagedKVCache (next_milestones.h:24-32) with device pools."""

    def __init__(self, config: PagedKVConfig, device="cuda"):
        import torch
        if config.head_dim != config.head_dim_value:
            raise ValueError("paged KV pools hold equal key and value widths")
        self.alloc = PageAllocator(config)
        self.config = config
        self.device = torch.device(device)
        self.lib = _abi.load()
        n, h, pt, d = config.num_pages, config.kv_heads, config.page_tokens, config.head_dim
        self.pool_dtype = F32 if config.pool_dtype == "f32" else BF16
        store = torch.float32 if self.pool_dtype == F32 else torch.int16
        self.k_pool = torch.zeros((n, h, pt, d), dtype=store, device=self.device)
        self.v_pool = torch.zeros((n, h, d, pt), dtype=store, device=self.device)
        self.table = torch.from_numpy(self.alloc.table_array()).to(self.device)

    # reference field names
    @property
    def length(self) -> int:
        return self.alloc.length

    @property
    def page_table(self) -> List[List[int]]:
        return self.alloc.page_table

    @property
    def free_pages(self) -> List[int]:
        return self.alloc.free_pages

    def _sync_table(self) -> None:
        import torch
        self.table.copy_(torch.from_numpy(self.alloc.table_array()))

    def dump(self) -> str:
        return (f"paged_kv batch={self.config.batch} kv_heads={self.config.kv_heads} "
                f"head_dim={self.config.head_dim} page_tokens={self.config.page_tokens} "
                f"capacity={self.config.capacity} length={self.length} "
                f"pages={[len(t) for t in self.page_table]} free={len(self.free_pages)}")


def make_paged_kv_cache(config: PagedKVConfig, device="cuda") -> PagedKVCache:
    """make_paged_kv_cache (next_milestones.cpp:472-484)."""
    return PagedKVCache(config, device)


def append_paged_kv(cache: PagedKVCache, keys, values, tokens: int, stream=None) -> None:
    """append_paged_kv (next_milestones.cpp:486-524): keys / values [B][Hkv][T][D]
    (fp32, or bf16 bits in int16) appended at the cache length, stored in the
    pools' dtype."""
    import torch
    c = cache.config
    shape = (c.batch, c.kv_heads, tokens, c.head_dim)
    keys = torch.as_tensor(keys, device=cache.device)
    values = torch.as_tensor(values, device=cache.device)
    if tokens <= 0 or keys.numel() != np.prod(shape) or values.numel() != np.prod(shape):
        if tokens <= 0:
            raise ValueError("paged KV capacity exceeded")
        raise ValueError("paged KV append shape mismatch")
    if keys.dtype != values.dtype or keys.dtype not in (torch.float32, torch.int16):
        raise ValueError("paged KV append: keys / values must both be fp32 or bf16 bits")
    dtype = F32 if keys.dtype == torch.float32 else BF16
    keys, values = keys.contiguous(), values.contiguous()
    cache.alloc.reserve(tokens)
    cache._sync_table()
    s = torch.cuda.current_stream(cache.device).cuda_stream if stream is None else stream
    check(cache.lib.sfg_hip_kv_append_pool_v1(
        keys.data_ptr(), values.data_ptr(), dtype, cache.k_pool.data_ptr(), cache.v_pool.data_ptr(),
        cache.pool_dtype, cache.table.data_ptr(), None, cache.length, 0, c.batch, c.kv_heads, tokens,
        c.head_dim, c.page_tokens, c.pages_per_seq, c.num_pages, s))
    torch.cuda.current_stream(cache.device).synchronize()
    cache.alloc.length += tokens


def truncate_paged_kv(cache: PagedKVCache, new_length: int) -> None:
    """truncate_paged_kv (next_milestones.cpp:542-552)."""
    cache.alloc.truncate(new_length)
    cache._sync_table()


def release_paged_kv_pages(cache: PagedKVCache, pages) -> None:
    """release_paged_kv_pages (next_milestones.cpp:527-540)."""
    cache.alloc.release(pages)


def gather_paged_kv(cache: PagedKVCache, stream=None):
    """gather_paged_kv (next_milestones.cpp:554-581): (keys, values) as fp32
    numpy [B][Hkv][length][D] in logical order."""
    import torch
    c = cache.config
    if cache.length <= 0:
        raise ValueError("cannot gather empty paged KV cache")
    keys = torch.empty((c.batch, c.kv_heads, cache.length, c.head_dim), dtype=torch.float32,
                       device=cache.device)
    values = torch.empty_like(keys)
    s = torch.cuda.current_stream(cache.device).cuda_stream if stream is None else stream
    check(cache.lib.sfg_hip_kv_gather_pool_v1(
        cache.k_pool.data_ptr(), cache.v_pool.data_ptr(), cache.pool_dtype, cache.table.data_ptr(),
        c.batch, c.kv_heads, cache.length, c.head_dim, c.page_tokens, c.pages_per_seq, c.num_pages,
        keys.data_ptr(), values.data_ptr(), s))
    torch.cuda.current_stream(cache.device).synchronize()
    return keys.cpu().numpy(), values.cpu().numpy()


def paged_decode_attention(cache: PagedKVCache, query, q_heads: int, seq_q: int = 1,
                           causal: bool = True, scale: float = 0.0, kv_splits: int = 0,
                           out_dtype=F32, stream=None) -> np.ndarray:
    """execute_paged_decode_attention (next_milestones.cpp:583-609) over the
    cache's pools: query [B][Hq][seq_q][D] fp32 attends over each sequence's
    cached tokens (query row i sees key j <= length - seq_q + i when causal,
    attention_compiler.cpp:68-72); returns [B][Hq][seq_q][D] fp32 (bf16 values
    when out_dtype is BF16) as numpy, through sfg_hip_attn_paged_v1."""
    import torch
    c = cache.config
    if cache.length <= 0:
        raise ValueError("cannot attend over an empty paged KV cache")
    if q_heads <= 0 or q_heads % c.kv_heads:
        raise ValueError("invalid attention configuration")
    q = torch.as_tensor(np.ascontiguousarray(query, np.float32)).to(cache.device)
    if q.numel() != c.batch * q_heads * seq_q * c.head_dim:
        raise ValueError("paged attention query shape mismatch")
    shape = (c.batch, q_heads, seq_q, c.head_dim)
    out = torch.empty(shape, dtype=torch.float32 if out_dtype == F32 else torch.int16, device=cache.device)
    ws_bytes = cache.lib.sfg_hip_attn_paged_workspace_v1(c.batch, q_heads, c.kv_heads, seq_q, c.head_dim,
                                                         cache.pool_dtype, cache.length, c.page_tokens,
                                                         kv_splits)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=cache.device)
    s = torch.cuda.current_stream(cache.device).cuda_stream if stream is None else stream
    check(cache.lib.sfg_hip_attn_paged_v1(
        q.data_ptr(), cache.k_pool.data_ptr(), cache.v_pool.data_ptr(), cache.pool_dtype,
        cache.table.data_ptr(), None, out.data_ptr(), out_dtype, c.batch, q_heads, c.kv_heads, seq_q,
        c.head_dim, c.page_tokens, c.pages_per_seq, c.num_pages, cache.length, int(causal), kv_splits,
        float(scale), 0, ws.data_ptr(), ws.numel(), s))
    torch.cuda.current_stream(cache.device).synchronize()
    res = out.cpu().numpy()
    if out_dtype != F32:
        res = (res.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    return res


def gather_plan_kv(plan, length: int, stream=None):
    """The first `length` tokens of a decoder plan's paged pools as fp32 numpy
    [B][Hkv][length][D] (gather_paged_kv over the plan's tables)."""
    import torch
    d = plan.desc
    keys = torch.empty((d.batch, d.kv_heads, length, d.head_dim), dtype=torch.float32, device=plan.device)
    values = torch.empty_like(keys)
    s = torch.cuda.current_stream(plan.device).cuda_stream if stream is None else stream
    check(plan.lib.sfg_hip_kv_gather_pool_v1(
        plan.t["k_pool"].data_ptr(), plan.t["v_pool"].data_ptr(), d.act_dtype, plan.t["page_table"].data_ptr(),
        d.batch, d.kv_heads, length, d.head_dim, d.page_tokens, d.pages_per_seq, d.num_pages,
        keys.data_ptr(), values.data_ptr(), s))
    torch.cuda.current_stream(plan.device).synchronize()
    return keys.cpu().numpy(), values.cpu().numpy()
