"""Page accounting shared by the KV-cache manager and the scheduler.

``PageAllocator`` is the protocol the reference scheduler programs against
(src/MoE/scheduler.py:101-111); ``pages_needed`` is scheduler.py:31-35.
``PagePool`` is the free-list logic of the reference engine's dynamic page
allocation (src/MoE/moe_engine.py:578-582, 4231-4297): a FIFO deque of
physical page ids, ``popleft`` on allocation, ``extend`` (append right) on
free, ``RuntimeError`` on exhaustion or on overflowing ``max_pages_per_seq``.
The one addition is ``free_order``: the initial free list may be given
explicitly (e.g. a seeded permutation, or a random subset of the pages) to
model a fragmented pool; the default is the reference's ``range(total_pages)``.
"""
from __future__ import annotations

import math
from collections import deque
from typing import Iterable, Optional, Protocol, runtime_checkable

__all__ = ["PageAllocator", "PagePool", "pages_needed"]


def pages_needed(seq_len: int, page_size: int) -> int:
    """KV pages for a sequence of ``seq_len`` tokens (scheduler.py:31-35)."""
    if seq_len <= 0:
        return 0
    return math.ceil(seq_len / page_size)


@runtime_checkable
class PageAllocator(Protocol):
    total_pages: int

    @property
    def pages_free(self) -> int: ...

    @property
    def pages_in_use(self) -> int: ...

    def alloc_pages(self, seq_id: int, n_pages: int) -> None: ...

    def free_seq(self, seq_id: int) -> None: ...

    def ensure_pages(self, seq_id: int, needed: int) -> None: ...

    def seq_pages(self, seq_id: int) -> int: ...


class PagePool:
    """Host-side page pool: free list + per-sequence page lists.

    ``alloc`` returns the newly assigned page ids so that the owner can mirror
    them into a device block table.
    """

    def __init__(self, total_pages: int, max_seqs: int, max_pages_per_seq: Optional[int] = None,
                 free_order: Optional[Iterable[int]] = None):
        if total_pages <= 0:
            raise ValueError("total_pages must be positive")
        self.total_pages = int(total_pages)
        self.max_seqs = int(max_seqs)
        self.max_pages_per_seq = max_pages_per_seq
        self._initial = None if free_order is None else [int(p) for p in free_order]
        if self._initial is not None:
            ids = self._initial
            if len(set(ids)) != len(ids) or any(p < 0 or p >= self.total_pages for p in ids):
                raise ValueError("free_order must hold distinct page ids in [0, total_pages)")
            # Pages left out of free_order start out owned elsewhere (a
            # pre-fragmented pool) and count as in use.
        self.reset()

    def reset(self) -> None:
        init = range(self.total_pages) if self._initial is None else self._initial
        self.free_pages: deque[int] = deque(init)
        self.seq_page_list: list[list[int]] = [[] for _ in range(self.max_seqs)]

    @property
    def pages_free(self) -> int:
        return len(self.free_pages)

    @property
    def pages_in_use(self) -> int:
        return self.total_pages - len(self.free_pages)

    def seq_pages(self, seq_id: int) -> int:
        return len(self.seq_page_list[seq_id])

    def alloc(self, seq_id: int, n_pages: int) -> tuple[int, list[int]]:
        """Assign ``n_pages`` more pages to ``seq_id``; returns (first logical
        page index, page ids).  Messages follow moe_engine.py:4241-4250."""
        if n_pages <= 0:
            return len(self.seq_page_list[seq_id]), []
        current = len(self.seq_page_list[seq_id])
        if self.max_pages_per_seq is not None and current + n_pages > self.max_pages_per_seq:
            raise RuntimeError(
                f"Cannot allocate {n_pages} pages for seq {seq_id}: "
                f"would exceed max_pages_per_seq={self.max_pages_per_seq} "
                f"(current={current})")
        if len(self.free_pages) < n_pages:
            raise RuntimeError(
                f"Cannot allocate {n_pages} pages for seq {seq_id}: "
                f"only {len(self.free_pages)} free pages remain "
                f"(budget={self.total_pages})")
        pages = [self.free_pages.popleft() for _ in range(n_pages)]
        self.seq_page_list[seq_id].extend(pages)
        return current, pages

    def release(self, seq_id: int) -> list[int]:
        """Return all pages of ``seq_id`` to the free list; returns them."""
        pages = self.seq_page_list[seq_id]
        if not pages:
            return []
        self.free_pages.extend(pages)
        self.seq_page_list[seq_id] = []
        return pages

    def detach(self, seq_id: int) -> list[int]:
        """Take the page list of ``seq_id`` away without freeing the pages
        (used while a swap-out still reads them)."""
        pages = self.seq_page_list[seq_id]
        self.seq_page_list[seq_id] = []
        return pages

    def give_back(self, pages: Iterable[int]) -> None:
        self.free_pages.extend(pages)
