"""Host-side page accounting (CPU only): the product's PagePool and the
page-pool API of PagedKVCache against the oracle's FifoPagePool, and the
invariants the reference checks in src/MoE/tests/test_dynamic_pages.py:38-136
(alloc / ensure / no overlap / free -> -1 / reset / exhaustion RuntimeError /
zero-alloc no-op) and src/MoE/tests/test_scheduling.py:458-488
(pages_in_use <= budget every step)."""
import random

import numpy as np
import pytest
import torch

from gpu_offloading_amd.allocator import PageAllocator, PagePool, pages_needed
from gpu_offloading_amd.kv_cache import PagedKVCache
from oracle import kv_oracle as orc


def test_pages_needed_matches_scheduler_formula():
    assert [pages_needed(n, 16) for n in (0, 1, 15, 16, 17, 32, 33)] == [0, 1, 1, 1, 2, 2, 3]
    assert pages_needed(-4, 16) == 0


def test_pagepool_matches_oracle_on_random_operations():
    rng = random.Random(0)
    order = list(range(40))
    rng.shuffle(order)
    pool = PagePool(40, 6, 12, free_order=order)
    ref = orc.FifoPagePool(40, 6, 12, free_order=order)
    bt = np.full((6, 12), -1, np.int32)
    for _ in range(500):
        op = rng.random()
        s = rng.randrange(6)
        if op < 0.6:
            n = rng.randrange(0, 5)
            err = None
            try:
                ref.alloc_pages(s, n)
            except RuntimeError as e:
                err = str(e)
            if err is None:
                cur, pages = pool.alloc(s, n)
                bt[s, cur:cur + len(pages)] = pages
            else:
                with pytest.raises(RuntimeError) as ei:
                    pool.alloc(s, n)
                assert str(ei.value) == err
        else:
            pages = pool.release(s)
            bt[s, :len(pages)] = -1
            ref.free_seq(s)
        assert pool.pages_free == ref.pages_free
        assert list(pool.free_pages) == list(ref.free)
        assert np.array_equal(bt, ref.block_table)


def cpu_cache(budget=12, max_seqs=3, max_seq_len=64, **kw):
    return PagedKVCache(1, 2, 8, max_seqs, max_seq_len, kv_page_budget=budget, device="cpu", **kw)


def test_kv_cache_page_api_invariants():
    c = cpu_cache(max_seq_len=160)
    assert isinstance(c, PageAllocator)
    assert c.pages_free == 12 and c.pages_in_use == 0
    c.alloc_pages(0, 3)
    c.ensure_pages(1, 2)
    c.ensure_pages(1, 1)                      # no-op
    c.alloc_pages(2, 0)                       # zero-alloc no-op
    assert (c.seq_pages(0), c.seq_pages(1), c.seq_pages(2)) == (3, 2, 0)
    bt = c.block_table.numpy()
    used = [p for row in bt for p in row if p >= 0]
    assert len(used) == len(set(used)) == 5   # no overlap between sequences
    assert bt[0, :3].tolist() == [0, 1, 2] and bt[1, :2].tolist() == [3, 4]
    c.free_seq(0)
    assert (c.block_table[0] == -1).all() and c.pages_free == 10
    assert c.seq_lens[0] == 0
    c.alloc_pages(2, 3)                       # FIFO: 5, 6, 7 before the freed 0, 1, 2
    assert c.block_table[2, :3].tolist() == [5, 6, 7]
    with pytest.raises(RuntimeError, match="free pages remain"):
        c.alloc_pages(0, 8)
    with pytest.raises(RuntimeError, match="max_pages_per_seq"):
        c.alloc_pages(2, 8)
    c.reset()
    assert c.pages_free == 12 and (c.block_table == -1).all()


def test_static_mode_has_identity_tables_and_no_allocator():
    c = PagedKVCache(1, 2, 8, max_seqs=3, max_seq_len=40, device="cpu")
    assert c.total_pages == 9
    assert c.block_table.tolist() == [[0, 1, 2], [3, 4, 5], [6, 7, 8]]
    assert c.seq_pages(1) == 3
    with pytest.raises(RuntimeError, match="dynamic pages"):
        c.alloc_pages(0, 1)


def test_gpu_only_operations_raise_on_a_cpu_cache():
    c = cpu_cache()
    with pytest.raises(RuntimeError, match="GPU-resident"):
        c.plan_decode([0])
    with pytest.raises(RuntimeError, match="GPU-resident"):
        c.slot_mapping([0], [1])


def test_planning_rejects_bad_seq_ids_and_oversized_sequences():
    """The host checks every planning call makes before it stages page
    indices: ids distinct rows of the table (a negative id would wrap in numpy
    indexing, a repeated one would size the page list past its device buffer),
    and no sequence longer than its block-table row."""
    c = cpu_cache(max_seqs=3, max_seq_len=64)
    for bad in ([-1], [3], [0, 0], [1, 2, 1]):
        with pytest.raises(ValueError, match="distinct"):
            c._check_seq_ids(bad)
    assert c._check_seq_ids([2, 0]).tolist() == [2, 0]
    assert c._check_seq_ids([]).tolist() == []
    c._check_page_counts(np.array([4, 0]))        # 64 tokens fill a row exactly
    with pytest.raises(RuntimeError, match="max_seq_len"):
        c._check_page_counts(np.array([1, 5]))


def test_scheduler_style_workload_keeps_pages_within_budget():
    """A continuous-batching loop in the scheduler's style (ensure_pages per
    decode token, free on completion, LIFO preemption when the pool is short):
    pages_in_use never exceeds the budget and everything is freed at the end."""
    rng = random.Random(1)
    budget = 20
    c = cpu_cache(budget=budget, max_seqs=4, max_seq_len=160)
    lens = {}
    waiting = [rng.randrange(1, 60) for _ in range(12)]
    running = []
    steps = 0
    while (waiting or running) and steps < 2000:
        steps += 1
        for s in list(running):
            if lens[s] >= 100 or rng.random() < 0.03:
                c.free_seq(s)
                running.remove(s)
                del lens[s]
        for s in list(running):
            need = pages_needed(lens[s] + 1, 16)
            while need - c.seq_pages(s) > c.pages_free and len(running) > 1:
                victim = running.pop()              # LIFO preemption -> recompute
                waiting.insert(0, lens.pop(victim))
                c.free_seq(victim)
            if s in running:
                c.ensure_pages(s, need)
                lens[s] += 1
        free_slots = [i for i in range(4) if i not in running]
        while waiting and free_slots and pages_needed(waiting[0], 16) <= c.pages_free:
            s = free_slots.pop(0)
            n = waiting.pop(0)
            c.alloc_pages(s, pages_needed(n, 16))
            lens[s] = n
            running.append(s)
        assert c.pages_in_use <= budget
        assert c.pages_in_use == sum(c.seq_pages(s) for s in range(4))
    for s in list(running):
        c.free_seq(s)
    assert c.pages_in_use == 0
