"""Host bookkeeping of the paged KV cache (no GPU): the reference's allocator
order and guards (next_milestones.cpp:472-552, test_schedforge.cpp:368-390)."""
from __future__ import annotations

import pytest

from schedforge_amd.kvcache import PageAllocator, PagedKVConfig


def test_reference_scenario_allocation_release_truncate():
    # test_schedforge.cpp:369-390 with 16-token pages: 23 tokens take two pages
    a = PageAllocator(PagedKVConfig(1, 2, 128, 128, 16, 48))
    assert a.free_pages == [0, 1, 2]
    a.reserve(23)
    a.length = 23
    assert a.page_table == [[2, 1]]          # popped from the back of the free list
    with pytest.raises(ValueError, match="active"):
        a.release([a.page_table[0][0]])
    before = len(a.page_table[0])
    a.truncate(3)
    assert a.length == 3 and len(a.page_table[0]) < before and a.free_pages
    assert a.free_pages == [0, 1]
    a.release([1])                           # already free: no duplicate
    assert a.free_pages == [0, 1]


def test_capacity_and_argument_guards():
    a = PageAllocator(PagedKVConfig(2, 1, 128, 128, 16, 40))
    assert a.config.pages_per_seq == 3 and a.config.num_pages == 6
    with pytest.raises(ValueError, match="capacity"):
        a.reserve(41)
    with pytest.raises(ValueError, match="capacity"):
        a.reserve(0)
    a.reserve(17)
    a.length = 17
    # each sequence owns its own pages
    assert [len(t) for t in a.page_table] == [2, 2]
    assert len({p for t in a.page_table for p in t}) == 4
    with pytest.raises(ValueError, match="truncation"):
        a.truncate(18)
    with pytest.raises(ValueError, match="invalid physical"):
        a.release([6])
    table = a.table_array()
    assert table.shape == (2, 3) and (table[:, 2] == -1).all()
    with pytest.raises(ValueError):
        PageAllocator(PagedKVConfig(1, 1, 128, 128, 16, 0))


def test_allocator_exhaustion_is_a_runtime_error():
    a = PageAllocator(PagedKVConfig(1, 1, 128, 128, 16, 32))
    a.free_pages.clear()
    with pytest.raises(RuntimeError, match="exhausted"):
        a.reserve(1)
