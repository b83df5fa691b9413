"""Ordering rules of block eviction / restore between the compute stream and
the swap's side streams.

A swap-out detaches a sequence's pages at once (block-table row -1, length
0), but its side stream still reads them until the device-to-host copy's
event completes; a swap-in allocates fresh pages at once, but its side
stream writes them until the restore's event completes.  ``SwapLedger``
keeps both kinds of pending work and enforces:

1. pages of a swap-out rejoin the free list only once its event has
   completed (``reclaim``; when the pool cannot otherwise serve an
   allocation, the oldest pending swap-out is waited for on the host, one at
   a time, and only as many as the allocation needs);
2. a restored sequence is used -- planned, gathered, swapped out again --
   only after the compute stream waited for its restore (``before_use``);
3. a sequence freed while its restore is in flight hands its pages on only
   after the compute stream waited for that restore (``on_free``), so the
   next owner's writes (on the compute stream, or on a side stream that
   waits for it) land after the restore's.

The precedent for the stream/event pattern is the reference's
replay_controller (src/MoE/replay_controller.py:184-185, 254-257, 313-345)
and the dense offload pipeline (src/dense/include/paged_offload_transformer.py:
394-418).  Events and streams are anything with ``query()`` /
``synchronize()`` and ``wait_event(ev)``: torch.cuda objects on the GPU, fakes
in the CPU tests.
"""
from __future__ import annotations

from typing import Any, Iterable, Sequence

__all__ = ["SwapLedger"]


class SwapLedger:
    def __init__(self):
        # (event, page ids to return, objects to keep alive until the event)
        self.pending_free: list[tuple[Any, list[int], list]] = []
        # sequence -> event of its restore still in flight
        self.pending_in: dict[int, Any] = {}

    @property
    def pending_pages(self) -> int:
        """Pages detached by swap-outs whose copies may still run: they are
        not owned by any sequence, and an allocation that needs them gets
        them (``reclaim`` waits for their copy)."""
        return sum(len(pages) for _, pages, _ in self.pending_free)

    def add_swap_out(self, event, pages: Sequence[int], keepalive: Iterable = ()) -> None:
        """``pages`` were detached by a swap-out whose copies end at ``event``."""
        self.pending_free.append((event, list(pages), list(keepalive)))

    def add_swap_in(self, event, seq_ids: Sequence[int], keepalive: Iterable = ()) -> None:
        """``seq_ids`` were restored by work that ends at ``event``."""
        self.pending_free.append((event, [], list(keepalive)))
        for s in seq_ids:
            self.pending_in[int(s)] = event

    def reclaim(self, pool, need: int = 0) -> None:
        """Give the pages of completed swap-outs back to ``pool``; wait on the
        host for the oldest pending ones only while ``pool`` holds fewer than
        ``need`` free pages."""
        still = []
        for ev, pages, keep in self.pending_free:
            if ev.query():
                pool.give_back(pages)
            else:
                still.append((ev, pages, keep))
        self.pending_free = still
        while self.pending_free and pool.pages_free < need:
            ev, pages, keep = self.pending_free.pop(0)
            ev.synchronize()
            pool.give_back(pages)

    def before_use(self, seq_ids: Iterable[int], stream) -> None:
        """Make ``stream`` wait for the pending restores of ``seq_ids``."""
        if not self.pending_in:
            return
        for s in seq_ids:
            ev = self.pending_in.pop(int(s), None)
            if ev is not None:
                stream.wait_event(ev)

    def on_free(self, seq_id: int, stream) -> None:
        """``seq_id`` is being freed: ``stream`` waits for its pending restore."""
        ev = self.pending_in.pop(int(seq_id), None)
        if ev is not None:
            stream.wait_event(ev)

    def clear(self) -> None:
        self.pending_free.clear()
        self.pending_in.clear()
