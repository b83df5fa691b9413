"""The swap event protocol on the CPU (gpu_offloading_amd/swap_ledger.py and
its use by PagedKVCache), with fake events and streams:

* pages detached by a swap-out rejoin the free list only after the
  swap-out's event completed -- never while its device-to-host copy may
  still read them; the host waits on the oldest pending swap-out only when
  an allocation cannot be served otherwise, and only as far as it needs;
* a restored sequence is planned / gathered / swapped again only after the
  compute stream waited for its restore, once, and only for the sequences
  used;
* a sequence freed while its restore is in flight makes the compute stream
  wait for that restore before its pages are handed on.
The GPU tests (test_gpu_cache_guards.py, test_gpu_cache_stress.py) run the
same rules with real streams."""
import pytest
import torch

from gpu_offloading_amd.allocator import PagePool
from gpu_offloading_amd.kv_cache import PagedKVCache
from gpu_offloading_amd.swap_ledger import SwapLedger


class FakeEvent:
    def __init__(self, name, done=False):
        self.name, self.done, self.synchronized = name, done, 0

    def query(self):
        return self.done

    def synchronize(self):
        self.synchronized += 1
        self.done = True


class FakeStream:
    def __init__(self):
        self.waited = []

    def wait_event(self, ev):
        self.waited.append(ev.name)


class RecordingPool(PagePool):
    """Fails if pages come back while the event of their swap-out is not done."""

    def __init__(self, *a, **kw):
        super().__init__(*a, **kw)
        self.events = {}      # page -> event of the swap-out that detached it

    def give_back(self, pages):
        for p in pages:
            ev = self.events.get(p)
            assert ev is None or ev.done, f"page {p} reused before {ev.name} completed"
        super().give_back(pages)


def _swap_out(ledger, pool, seq, ev):
    pages = pool.detach(seq)
    for p in pages:
        pool.events[p] = ev
    ledger.add_swap_out(ev, pages)
    return pages


def test_swapped_out_pages_wait_for_their_copy():
    pool = RecordingPool(8, 4, 8)
    led = SwapLedger()
    pool.alloc(0, 6)
    ev = FakeEvent("out0")
    pages = _swap_out(led, pool, 0, ev)
    assert pool.pages_free == 2
    led.reclaim(pool, need=2)                 # enough free pages: no wait, nothing back
    assert ev.synchronized == 0 and pool.pages_free == 2
    led.reclaim(pool, need=3)                 # short: wait for the copy, then reuse
    assert ev.synchronized == 1 and pool.pages_free == 8
    assert sorted(list(pool.free_pages)[2:]) == sorted(pages)


def test_completed_swap_outs_return_without_waiting():
    pool = RecordingPool(8, 4, 8)
    led = SwapLedger()
    pool.alloc(0, 3)
    ev = FakeEvent("out0")
    _swap_out(led, pool, 0, ev)
    led.reclaim(pool)
    assert pool.pages_free == 5 and led.pending_free
    ev.done = True                            # the copy finished on the device
    led.reclaim(pool)
    assert pool.pages_free == 8 and not led.pending_free and ev.synchronized == 0


def test_host_waits_on_the_oldest_swap_outs_only_as_needed():
    pool = RecordingPool(9, 4, 9)
    led = SwapLedger()
    evs = []
    for s in range(3):
        pool.alloc(s, 3)
        evs.append(FakeEvent(f"out{s}"))
        _swap_out(led, pool, s, evs[-1])
    assert pool.pages_free == 0
    led.reclaim(pool, need=4)                 # two swap-outs cover four pages
    assert [e.synchronized for e in evs] == [1, 1, 0]
    assert pool.pages_free == 6 and len(led.pending_free) == 1


def test_restored_sequences_are_used_after_their_restore():
    led = SwapLedger()
    ev_a, ev_b = FakeEvent("in_a"), FakeEvent("in_b")
    led.add_swap_in(ev_a, [1, 2])
    led.add_swap_in(ev_b, [5])
    cur = FakeStream()
    led.before_use([0, 2], cur)               # sequence 2 was restored by ev_a
    assert cur.waited == ["in_a"]
    led.before_use([2, 5, 1], cur)            # 2 already waited for; 5 and 1 now
    assert cur.waited == ["in_a", "in_b", "in_a"]
    led.before_use([1, 2, 5], cur)
    assert cur.waited == ["in_a", "in_b", "in_a"]
    assert not led.pending_in


def test_free_during_restore_waits_for_it():
    led = SwapLedger()
    ev = FakeEvent("in3")
    led.add_swap_in(ev, [3])
    cur = FakeStream()
    led.on_free(4, cur)                        # nothing pending for 4
    assert cur.waited == []
    led.on_free(3, cur)
    assert cur.waited == ["in3"] and 3 not in led.pending_in


def test_paged_kv_cache_follows_the_protocol(monkeypatch):
    """The same rules through PagedKVCache's page API on a CPU cache: an
    allocation that needs a swapped-out sequence's pages waits for its copy
    first; free_seq during a restore orders the compute stream after it."""
    cache = PagedKVCache(1, 2, 8, max_seqs=4, max_seq_len=128, kv_page_budget=8,
                         device="cpu")
    cache._pool.__class__ = RecordingPool
    cache._pool.events = {}
    cache.alloc_pages(0, 6)
    ev = FakeEvent("out0")
    _swap_out(cache._swaps, cache._pool, 0, ev)     # the bookkeeping swap_out does
    # the victim's pages count as free for the scheduler at once (an
    # allocation that needs them waits for the copy), as after free_seq
    assert cache.pages_free == 8 and cache.pages_in_use == 0
    assert cache._swaps.pending_pages == 6
    cache.alloc_pages(1, 2)                          # served by the free pages
    assert ev.synchronized == 0
    assert cache.pages_free == 6 and cache.pages_in_use == 2
    cache.alloc_pages(2, 3)                          # needs the swapped-out pages
    assert ev.synchronized == 1 and cache.seq_pages(2) == 3
    cur = FakeStream()
    monkeypatch.setattr(torch.cuda, "current_stream", lambda *a, **k: cur)
    ev_in = FakeEvent("in1")
    cache._swaps.add_swap_in(ev_in, [1])
    cache.free_seq(1)
    assert cur.waited == ["in1"] and cache.seq_pages(1) == 0
    cache.reset()
    assert not cache._swaps.pending_free and not cache._swaps.pending_in
