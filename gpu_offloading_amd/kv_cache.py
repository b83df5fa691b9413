"""The paged KV cache of the reference MoE engine, MI355X-native.

``PagedKVCache`` is the KV-cache subset of ``MoEEngine``
(src/MoE/moe_engine.py): the per-layer ``k_cache`` / ``v_cache`` tensors
(:488-500), the block table (:504-519), ``seq_lens`` with its host mirror
(:535-539), the dynamic page pool and its API (:578-582, 4185-4297),
``kv_snapshot`` / ``kv_restore`` / ``fill_kv_random`` (:4152-4183), the slot
mapping and decode planning of a step (:1896-1955, 3475-3556), the
continuation-prefill planning (:1678-1751, 3649-3727) and the kernels called
per layer: the KV append (:2343-2347), decode attention (:3907-3909) and
paged prefill attention (:3939-3941).  It also adds the swap API the engine lacks (block eviction to
pinned host memory and restore, on a side stream).

All arithmetic runs in libkvc.so; this module only does host bookkeeping,
small H2D copies of metadata, and stream/event ordering.
"""
from __future__ import annotations

import collections
import math
from dataclasses import dataclass, field
from typing import Iterable, Optional, Sequence

import numpy as np
import torch

from . import _lib, hostmem, ops
from .allocator import PagePool, pages_needed
from .decode import BatchDecodeWithPagedKVCacheWrapper
from .prefill import BatchPrefillWithPagedKVCacheWrapper
from .swap_ledger import SwapLedger

__all__ = ["PagedKVCache", "SwapHandle"]


@dataclass
class SwapHandle:
    """Sequences whose KV lives in pinned host memory after ``swap_out``."""

    seq_ids: list[int]
    seq_lens: list[int]
    num_pages: list[int]
    src_block_ids: torch.Tensor          # device int32, evicted ids (concatenated)
    host: torch.Tensor                   # pinned uint8 [layers, n, 2, block_bytes]
    out_event: torch.cuda.Event          # D2H complete
    out_start: Optional[torch.cuda.Event] = None   # side stream reached the swap-out
    in_event: Optional[torch.cuda.Event] = None
    in_start: Optional[torch.cuda.Event] = None
    dst_block_ids: Optional[torch.Tensor] = None
    restored: bool = False
    num_bytes: int = 0                   # bytes over the host link each way
    _keepalive: list = field(default_factory=list)

    @property
    def num_blocks(self) -> int:
        return int(self.src_block_ids.numel())

    @property
    def bytes_per_direction(self) -> int:
        """Bytes that cross the host link each way (all layers, K and V)."""
        return self.num_bytes

    def out_seconds(self) -> float:
        """Side-stream time of the swap-out (gathers + D2H copies); call after
        ``out_event`` completed."""
        return self.out_start.elapsed_time(self.out_event) * 1e-3

    def in_seconds(self) -> float:
        """Side-stream time of the swap-in (H2D copies + scatters)."""
        return self.in_start.elapsed_time(self.in_event) * 1e-3


class PagedKVCache:
    """Per-layer paged K/V storage, block table and page pool.

    Arguments follow ``MoEEngine.__init__`` (moe_engine.py:79-95, 291-301):
    ``total_pages = kv_page_budget`` in dynamic mode, otherwise
    ``max_seqs * ceil(max_seq_len / page_size)`` with identity block-table rows.
    ``free_page_order`` optionally replaces the initial FIFO free list
    ``range(total_pages)`` (e.g. a seeded permutation for a fragmented pool).
    """

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, max_seqs: int,
                 max_seq_len: int, *, num_qo_heads: Optional[int] = None, page_size: int = 16,
                 kv_page_budget: Optional[int] = None, dtype: torch.dtype = torch.bfloat16,
                 device: str | torch.device = "cuda",
                 free_page_order: Optional[Iterable[int]] = None,
                 workspace_bytes: int = 128 * 1024 * 1024,
                 staging_bytes: int = 256 * 1024 * 1024,
                 num_segments: Optional[int] = None):
        if page_size != 16:
            raise ValueError("page_size must be 16 (the engine's page size)")
        self.device = torch.device(device)
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.num_heads = num_qo_heads if num_qo_heads is not None else num_kv_heads
        self.head_dim = head_dim
        self.page_size = page_size
        self.dtype = dtype
        self.max_seqs = max_seqs
        self.max_seq_len = max_seq_len
        self.max_pages_per_seq = math.ceil(max_seq_len / page_size)
        self._dynamic_pages = kv_page_budget is not None
        self.total_pages = kv_page_budget if self._dynamic_pages else max_seqs * self.max_pages_per_seq

        # One tensor per layer in FlashInfer's paged "NHD" layout
        # [pages, 2, page_size, Hkv, D]: a page's K block and V block are
        # adjacent (64 KB for Mixtral), so a decode touches half as many
        # distinct memory pages as with separate K and V tensors (cfg2 step
        # 3.23 -> 3.12 ms).  k_cache[l] / v_cache[l] are the engine's
        # [pages, page_size, Hkv, D] caches, as views.
        self.kv_cache = [torch.zeros((self.total_pages, 2, page_size, num_kv_heads, head_dim),
                                     dtype=dtype, device=self.device) for _ in range(num_layers)]
        self.k_cache = [t[:, 0] for t in self.kv_cache]
        self.v_cache = [t[:, 1] for t in self.kv_cache]
        # Each layer's cache arguments of a decode launch (pointers, block and
        # token strides, blocks): fixed for the cache's life.
        self._layer_kv = [(k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), k.shape[0])
                          for k, v in zip(self.k_cache, self.v_cache)]

        if self._dynamic_pages:
            self._bt = torch.full((max_seqs, self.max_pages_per_seq), -1,
                                  dtype=torch.int32, device=self.device)
        else:
            self._bt = torch.arange(max_seqs * self.max_pages_per_seq, dtype=torch.int32,
                                    device=self.device).view(max_seqs, self.max_pages_per_seq)
        # Block-table writes of a GPU cache wait here (flat position -> page
        # id, last write wins) until the next decode step uploads them with
        # the rest of its metadata, or ``block_table`` is read.
        self._bt_pending: dict[int, int] = {}
        # slots of the step set up by prepare_decode_step (append_and_decode)
        self._step_slots: Optional[torch.Tensor] = None
        # device copy of a decode step's metadata image (reused every step),
        # its slot mapping, and the streams that read them since the last
        # upload (handle -> stream; the next upload waits for each)
        self._step_dev: Optional[torch.Tensor] = None
        self._slots_dev: Optional[torch.Tensor] = None
        self._step_views = None
        self._step_layout = _lib.KvcDecodeStepLayout()
        self._step_handle: Optional[int] = None
        self._step_stream_obj = None
        self._step_users: dict = {}
        self._mixed_step_buf: Optional[torch.Tensor] = None
        self.seq_lens = torch.zeros(max_seqs, dtype=torch.int32, device=self.device)
        self._seq_lens_cpu = torch.zeros(max_seqs, dtype=torch.int32)
        self._pool = PagePool(self.total_pages, max_seqs, self.max_pages_per_seq,
                              free_order=free_page_order) if self._dynamic_pages else None

        self._workspace_bytes = workspace_bytes
        self._segments = num_segments
        self._decode_wrapper: Optional[BatchDecodeWithPagedKVCacheWrapper] = None
        if self.device.type == "cuda":
            self._init_step_buffers()

        # Pinned images of the step metadata, reused round-robin: a fresh
        # pinned tensor per step costs a host allocation (and a wait) whenever
        # the host runs ahead of the GPU, as it does when the layers are
        # replayed from a graph.  Each slot: [buffer, event of its last copy].
        self._meta_ring: list[list] = [[None, None] for _ in range(self._META_RING)]
        self._meta_step = 0
        self._meta_events: collections.deque = collections.deque()

        self._staging_bytes = staging_bytes
        self._staging: Optional[torch.Tensor] = None
        self._staging_free: list[Optional[torch.cuda.Event]] = [None, None]
        self._swap_stream: Optional[torch.cuda.Stream] = None
        self._copy_stream: Optional[torch.cuda.Stream] = None
        self._swap_warm = False   # reserve_swap's copy-path warm-up done
        self._swaps = SwapLedger()   # swap-outs / restores still in flight

    def _init_step_buffers(self) -> None:
        """Decode workspace + wrapper and the device page-index buffer
        (moe_engine.py:541-575).  Only a GPU cache has them; a CPU-resident
        instance supports the page-pool API alone.  Per-step host metadata is
        staged through fresh pinned tensors from torch's caching host
        allocator, which keeps each one alive until its async copy is done,
        so planning never waits for the GPU."""
        self._workspace_buf = torch.zeros(self._workspace_bytes, dtype=torch.uint8,
                                          device=self.device)
        self._decode_wrapper = BatchDecodeWithPagedKVCacheWrapper(
            self._workspace_buf, kv_layout="NHD", use_cuda_graph=False,
            num_segments=self._segments)
        self._plan_indices_gpu = torch.zeros(self.max_seqs * self.max_pages_per_seq,
                                             dtype=torch.int32, device=self.device)
        self._prefill_wrapper = BatchPrefillWithPagedKVCacheWrapper(self._workspace_buf,
                                                                    kv_layout="NHD")
        self._prefill_indices_gpu = torch.zeros(self.max_seqs * self.max_pages_per_seq,
                                                dtype=torch.int32, device=self.device)

    def _to_device(self, arr) -> torch.Tensor:
        """Async H2D of a small host array through a fresh pinned buffer."""
        t = torch.as_tensor(arr)
        return t.pin_memory().to(self.device, non_blocking=True)

    def _lens_to_device(self) -> None:
        """Refresh the device mirror of the lengths from the host copy."""
        if self.device.type == "cuda":
            self.seq_lens.copy_(self._seq_lens_cpu.pin_memory(), non_blocking=True)
        else:
            self.seq_lens.copy_(self._seq_lens_cpu)

    @property
    def block_table(self) -> torch.Tensor:
        """``[max_seqs, max_pages_per_seq]`` int32 physical page ids (-1 for
        none), on the cache's device, with every earlier write applied."""
        self._flush_block_table()
        return self._bt

    def _bt_write(self, seq_id: int, start: int, pages) -> None:
        """``block_table[seq_id, start:start+len(pages)] = pages`` (an int or
        a sequence), deferred on a GPU cache."""
        if isinstance(pages, int):
            raise TypeError("pages must be a sequence")
        if self.device.type != "cuda":
            self._bt[seq_id, start:start + len(pages)] = torch.as_tensor(pages, dtype=torch.int32)
            return
        base = seq_id * self.max_pages_per_seq + start
        for j, p in enumerate(pages):
            self._bt_pending[base + j] = int(p)

    def _peek_bt_pending(self):
        """(positions int64, values int32) of the pending writes, or None.
        Callers clear ``_bt_pending`` once the writes are enqueued, so that an
        error on the way leaves them pending."""
        if not self._bt_pending:
            return None
        pos = np.fromiter(self._bt_pending.keys(), dtype=np.int64, count=len(self._bt_pending))
        val = np.fromiter(self._bt_pending.values(), dtype=np.int32, count=len(self._bt_pending))
        return pos, val

    def _flush_block_table(self) -> None:
        pend = self._peek_bt_pending()
        if pend is None:
            return
        pos, val = pend
        both = np.concatenate([pos, val.astype(np.int64)])
        d = self._to_device(both)
        self._bt.view(-1).scatter_(0, d[:len(pos)], d[len(pos):].to(torch.int32))
        self._bt_pending.clear()

    def _require_gpu(self) -> None:
        if self._decode_wrapper is None:
            raise RuntimeError("this operation needs a GPU-resident PagedKVCache (device='cuda')")

    # ------------------------------------------------------------ page pool
    def _require_dynamic(self) -> None:
        if not self._dynamic_pages:
            raise RuntimeError("page allocation needs dynamic pages (construct with kv_page_budget)")

    @property
    def _seq_page_list(self) -> list[list[int]]:
        self._require_dynamic()
        return self._pool.seq_page_list

    @property
    def _free_pages(self):
        self._require_dynamic()
        return self._pool.free_pages

    def alloc_pages(self, seq_id: int, n_pages: int) -> None:
        """moe_engine.py:4231-4259: take n_pages from the free list (FIFO) and
        write them to ``block_table[seq_id, current:current+n]``."""
        self._require_dynamic()
        if n_pages <= 0:
            return
        self._reclaim(need=n_pages)
        current, pages = self._pool.alloc(seq_id, n_pages)
        self._bt_write(seq_id, current, pages)

    def free_seq_pages(self, seq_id: int) -> None:
        """moe_engine.py:4261-4273: pages back to the free list, row -> -1."""
        self._require_dynamic()
        pages = self._pool.release(seq_id)
        if pages:
            self._bt_write(seq_id, 0, [-1] * len(pages))

    def ensure_pages(self, seq_id: int, needed_pages: int) -> None:
        """moe_engine.py:4275-4283: grow seq_id to needed_pages (no-op if enough)."""
        self._require_dynamic()
        current = self._pool.seq_pages(seq_id)
        if needed_pages > current:
            self.alloc_pages(seq_id, needed_pages - current)

    @property
    def pages_free(self) -> int:
        """Pages an allocation can take: the free list plus the pages of
        swap-outs still copying (``alloc_pages`` waits for those copies when
        it needs their pages).  So a scheduler sees a swapped-out victim's
        pages as freed at once, as after the reference's ``free_seq``
        (scheduler.py:329-333)."""
        self._require_dynamic()
        return self._pool.pages_free + self._swaps.pending_pages

    @property
    def pages_in_use(self) -> int:
        """Pages owned by sequences (``total_pages - pages_free``)."""
        self._require_dynamic()
        return self._pool.pages_in_use - self._swaps.pending_pages

    def seq_pages(self, seq_id: int) -> int:
        if not self._dynamic_pages:
            return self.max_pages_per_seq
        return self._pool.seq_pages(seq_id)

    def free_seq(self, seq_id: int) -> None:
        """moe_engine.py:4212-4227: seq_len -> 0 and (dynamic) pages freed.

        A restore of this sequence still in flight on the side stream keeps
        writing its pages: the current stream first waits for it, so that
        whoever is given the pages next (an append on the current stream, a
        swap on the side stream, which waits for the current one) writes
        after the restore."""
        if self._swaps.pending_in:
            self._swaps.on_free(seq_id, torch.cuda.current_stream(self.device))
        self._seq_lens_cpu[seq_id] = 0
        self.seq_lens[seq_id] = 0
        if self._dynamic_pages:
            self.free_seq_pages(seq_id)

    def reset(self) -> None:
        """moe_engine.py:4185-4210: zero lengths and caches, refill the pool."""
        self.synchronize_swaps()
        self._step_slots = None
        self.seq_lens.zero_()
        self._seq_lens_cpu.zero_()
        for kc, vc in zip(self.k_cache, self.v_cache):
            kc.zero_()
            vc.zero_()
        if self._dynamic_pages:
            self._pool.reset()
            self._bt_pending.clear()
            self._bt.fill_(-1)
        self._swaps.clear()

    # ----------------------------------------------------- snapshot / fill
    def fill_kv_random(self, std: float = 0.01, generator: Optional[torch.Generator] = None) -> None:
        for kc, vc in zip(self.k_cache, self.v_cache):
            kc.normal_(0, std, generator=generator)
            vc.normal_(0, std, generator=generator)

    def kv_snapshot(self):
        return ([kc.clone() for kc in self.k_cache], [vc.clone() for vc in self.v_cache])

    def kv_restore(self, snapshot) -> None:
        a, b = snapshot
        for kc, s in zip(self.k_cache, a):
            kc.copy_(s)
        for vc, s in zip(self.v_cache, b):
            vc.copy_(s)

    # --------------------------------------------------------- step metadata
    def _check_seq_ids(self, seq_ids: Sequence[int]) -> np.ndarray:
        """``seq_ids`` as int64, after checking they are distinct rows of the
        block table (a negative id would wrap in numpy indexing, and a
        repeated one could size the page list past its device buffer)."""
        ids = np.asarray(seq_ids, dtype=np.int64).reshape(-1)
        n = len(ids)
        if n and (ids.min() < 0 or ids.max() >= self.max_seqs
                  or (n > 1 and (len(set(ids.tolist())) if n <= 64 else len(np.unique(ids))) != n)):
            raise ValueError(f"seq_ids must be distinct and in [0, {self.max_seqs})")
        return ids

    def _check_page_counts(self, nblk: np.ndarray) -> None:
        """Every planned sequence fits its block-table row, so the flattened
        page list of distinct sequences fits the device index buffer."""
        if len(nblk) and int(nblk.max()) > self.max_pages_per_seq:
            raise RuntimeError(f"a sequence holds more than max_seq_len "
                               f"({self.max_pages_per_seq * self.page_size}) tokens")

    def _sync_seqs(self, seq_ids: Sequence[int]) -> None:
        """Order the current stream after pending swap-ins of these sequences."""
        if self._swaps.pending_in:
            self._swaps.before_use(seq_ids, torch.cuda.current_stream(self.device))

    def slot_mapping(self, seq_ids: Sequence[int], num_new_tokens: Sequence[int],
                     graph_n: Optional[int] = None) -> torch.Tensor:
        """Slots of the next tokens of each sequence (positions continue from
        ``seq_lens``), padded with -1 to ``graph_n`` tokens, computed on the
        device (moe_engine.py:3475-3541).  Does not advance ``seq_lens``."""
        self._require_gpu()
        r = len(seq_ids)
        n = int(sum(num_new_tokens))
        graph_n = n if graph_n is None else graph_n
        out = torch.empty(graph_n, dtype=torch.int64, device=self.device)
        if r == 0 or graph_n == 0:
            out.fill_(-1)
            return out
        ids = self._to_device(np.asarray(seq_ids, dtype=np.int32))
        qsl = np.zeros(r + 1, dtype=np.int32)
        np.cumsum(np.asarray(num_new_tokens, dtype=np.int32), out=qsl[1:])
        qsl_d = self._to_device(qsl)
        # Safety sync of the device lengths from the host mirror (the engine
        # does the same at moe_engine.py:3511).
        self._lens_to_device()
        ops.compute_slot_mapping(self.block_table, ids, qsl_d, self.seq_lens, n, out,
                                 block_size=self.page_size)
        return out

    def advance(self, seq_ids: Sequence[int], num_new_tokens: Sequence[int] | int = 1) -> None:
        """``_seq_lens_cpu[sid] += n`` (and the device mirror)."""
        lens = self._seq_lens_cpu.numpy()
        if isinstance(num_new_tokens, int):
            num_new_tokens = [num_new_tokens] * len(seq_ids)
        for sid, n in zip(seq_ids, num_new_tokens):
            lens[int(sid)] += int(n)
        self._lens_to_device()

    def plan_decode(self, seq_ids: Sequence[int]) -> None:
        """moe_engine.py:1896-1955: indptr / last_page_len on the host,
        page indices flattened on the device, then ``wrapper.plan``."""
        self._require_gpu()
        self._step_slots = None
        ids = self._check_seq_ids(seq_ids)
        b = len(ids)
        if b == 0:
            return
        self._sync_seqs(seq_ids)
        lens = self._seq_lens_cpu.numpy()[ids].astype(np.int32)
        nblk = (lens + self.page_size - 1) // self.page_size
        indptr = np.zeros(b + 1, dtype=np.int32)
        np.cumsum(nblk, out=indptr[1:])
        lpl = lens % self.page_size
        lpl = np.where((lpl == 0) & (lens != 0), self.page_size, lpl).astype(np.int32)
        self._check_page_counts(nblk)
        indptr_d = self._to_device(indptr)
        ids_d = self._to_device(ids.astype(np.int32))
        ops.copy_page_indices(self.block_table, indptr_d, self._plan_indices_gpu, seq_ids=ids_d)
        total = int(indptr[b])
        self._decode_wrapper.plan(
            torch.from_numpy(indptr), self._plan_indices_gpu[:total], torch.from_numpy(lpl),
            num_qo_heads=self.num_heads, num_kv_heads=self.num_kv_heads, head_dim=self.head_dim,
            page_size=self.page_size, pos_encoding_mode="NONE", q_data_type=self.dtype)

    def plan_prefill(self, seq_ids: Sequence[int], chunk_lens: Sequence[int]) -> None:
        """moe_engine.py:3649-3727: plan paged-KV prefill for continuation
        chunks whose K/V are already appended and counted in ``seq_lens``
        (query rows are the last ``chunk_lens[i]`` tokens of each sequence,
        causal against everything cached)."""
        self._require_gpu()
        self._step_slots = None
        ids = self._check_seq_ids(seq_ids)
        b = len(ids)
        if len(chunk_lens) != b:
            raise ValueError("one chunk length per sequence")
        self._sync_seqs(seq_ids)
        lens = self._seq_lens_cpu.numpy()[ids].astype(np.int64)
        clen = np.asarray(chunk_lens, dtype=np.int64)
        if (clen < 0).any() or (clen > lens).any():
            raise ValueError("a chunk must be part of its sequence's cached tokens")
        nblk = (lens + self.page_size - 1) // self.page_size
        kv_indptr = np.zeros(b + 1, dtype=np.int32)
        np.cumsum(nblk, out=kv_indptr[1:])
        qo_indptr = np.zeros(b + 1, dtype=np.int32)
        np.cumsum(clen, out=qo_indptr[1:])
        lpl = lens % self.page_size
        lpl = np.where((lpl == 0) & (lens != 0), self.page_size, lpl).astype(np.int32)
        self._check_page_counts(nblk)
        ops.copy_page_indices(self.block_table, self._to_device(kv_indptr),
                              self._prefill_indices_gpu, seq_ids=self._to_device(ids.astype(np.int32)))
        total = int(kv_indptr[b])
        self._prefill_wrapper.plan(
            torch.from_numpy(qo_indptr), torch.from_numpy(kv_indptr),
            self._prefill_indices_gpu[:total], torch.from_numpy(lpl),
            num_qo_heads=self.num_heads, num_kv_heads=self.num_kv_heads,
            head_dim_qk=self.head_dim, page_size=self.page_size, causal=True,
            q_data_type=self.dtype)

    def prepare_prefill_chunk(self, seq_ids: Sequence[int], chunk_lens: Sequence[int]) -> torch.Tensor:
        """Setup of a continuation-prefill step (moe_engine.py:1678-1751):
        slot mapping of the chunk's tokens from the current lengths, then
        ``seq_lens += chunk``, then the prefill plan.  Pages must already
        cover the chunk.  Returns the chunk's slot mapping for ``append``."""
        self._require_gpu()
        self._sync_seqs(seq_ids)
        slots = self.slot_mapping(seq_ids, chunk_lens)
        self.advance(seq_ids, list(chunk_lens))
        self.plan_prefill(seq_ids, chunk_lens)
        return slots

    def prefill(self, layer: int, q: torch.Tensor, out: Optional[torch.Tensor] = None,
                return_lse: bool = False):
        """Causal attention of the planned chunks' queries ``[sum(chunk), Hq, D]``
        over the paged cache of ``layer`` (moe_engine.py:3939-3941)."""
        self._require_gpu()
        self._step_stream_for_call()
        return self._prefill_wrapper.run(q, (self.k_cache[layer], self.v_cache[layer]),
                                         out=out, return_lse=return_lse)

    def prepare_decode_step(self, seq_ids: Sequence[int], graph_n: Optional[int] = None) -> torch.Tensor:
        """Setup of a pure-decode step in the engine's order
        (moe_engine.py:2655-2695, 3511-3556): slot mapping from the current
        lengths, then ``seq_lens += 1``, then plan.  Pages must already cover
        the new token (the scheduler's ``ensure_pages``).

        The device work is one launch (``kvc_decode_step_setup``) on the
        current stream.  The returned slot mapping (int64, -1 padded to
        ``graph_n``) lives in a buffer the cache reuses: it holds this step's
        slots until the next ``prepare_decode_step``, like the engine's static
        slot-mapping buffer.  The step's metadata also lives in a reused
        buffer; eager ``decode``/``append_and_decode`` calls on another stream
        are ordered after this setup, and the next setup after them.  A
        graph replay of the step's launches must run on this call's stream
        (or the caller orders the streams)."""
        self._require_gpu()
        b = len(seq_ids)
        graph_n = b if graph_n is None else graph_n
        self._step_slots = None
        if b == 0 or graph_n < b:
            # Nothing to plan, or an error for slot_mapping to report.
            slots = self.slot_mapping(seq_ids, [1] * b, graph_n)
            return slots
        ids = self._check_seq_ids(seq_ids)
        self._sync_seqs(seq_ids)
        lens_all = self._seq_lens_cpu.numpy()
        ms, ps = self.max_seqs, self.page_size
        lens = lens_all[ids].astype(np.int32) + 1
        if int(lens.max()) > self.max_pages_per_seq * ps:
            raise RuntimeError(f"a sequence would exceed max_seq_len ({self.max_pages_per_seq * ps})")
        if self._dynamic_pages:
            short = [int(s) for s, n in zip(ids, lens)
                     if self._pool.seq_pages(int(s)) * ps < n]
            if short:
                raise RuntimeError(f"sequences {short} have no page for the new token "
                                   "(ensure_pages first)")

        # One pinned int32 image of the step's metadata, read by one setup
        # kernel that also writes its device copy into the cache's step
        # buffer (the same device memory every step, so a decode launch
        # captured in a graph reads the new plan when replayed):
        #   decode schedule (cap, 16-byte aligned) | ids[b] | positions[b]
        #   | kv_indptr[b+1] | last_page_len[b] | lens_after[ms]
        #   | block-table positions (int64) | page ids
        pend = self._peek_bt_pending()
        u = 0 if pend is None else len(pend[0])
        w = self._decode_wrapper
        cap = w._plan_capacity(b)
        while True:
            o_ids = cap
            o_pos = o_ids + b
            o_ip = o_pos + b
            o_lpl = o_ip + b + 1
            o_la = o_lpl + b
            o_bpos = (o_la + ms + 1) // 2 * 2
            o_bval = o_bpos + 2 * u
            n = o_bval + u
            hs, h = self._host_image_np(n)
            h[o_ids:o_pos] = ids
            h[o_pos:o_ip] = lens_all[ids]
            nblk = (lens + ps - 1) // ps
            h[o_ip] = 0
            np.cumsum(nblk, out=h[o_ip + 1:o_ip + b + 1])
            h[o_lpl:o_lpl + b] = (lens - 1) % ps + 1     # lens >= 1
            h[o_la:o_la + ms] = lens_all
            h[o_la + ids] += 1
            if u:
                h[o_bpos:o_bpos + 2 * u].view(np.int64)[:] = pend[0]
                h[o_bval:o_bval + u] = pend[1]
            sched = w._schedule_into(h[o_ip:o_ip + b + 1], h[o_lpl:o_lpl + b], b,
                                     self.num_heads, self.num_kv_heads, self.head_dim, ps,
                                     h[0:cap])
            if sched.plan_ints <= cap:
                break
            cap = (sched.plan_ints + 3) // 4 * 4

        sh = self._claim_step_buffer()
        self._mixed_step_buf = None
        if self._step_dev is None or self._step_dev.numel() < n:
            # grows rarely (more requests or block-table writes than before);
            # a graph captured before must then be captured again
            self._step_dev = torch.empty(2 * max(n, 0 if self._step_dev is None
                                                 else self._step_dev.numel()),
                                         dtype=torch.int32, device=self.device)
        if self._slots_dev is None or self._slots_dev.numel() < graph_n:
            self._slots_dev = torch.empty(2 * graph_n, dtype=torch.int64, device=self.device)
        # Views of the step buffers, made again only when a shape changes.
        vk = (self._step_dev.data_ptr(), self._slots_dev.data_ptr(), cap, b, graph_n)
        if self._step_views is None or self._step_views[0] != vk:
            dm = self._step_dev
            self._step_views = (vk, dm[0:cap], dm[o_ip:o_lpl], dm[o_lpl:o_lpl + b],
                                self._slots_dev[:graph_n], self._slots_dev[:b])
        _, plan_v, indptr_v, lpl_v, slots, step_slots = self._step_views
        lay = self._step_layout
        lay.plan_ints = int(sched.plan_ints)   # the plan's unused capacity is not sent
        lay.tail_begin, lay.tail_end = cap, n
        lay.ids, lay.positions, lay.indptr, lay.lens_after = o_ids, o_pos, o_ip, o_la
        lay.bt_pos, lay.bt_val = o_bpos, o_bval
        lay.num_reqs, lay.num_bt_writes, lay.max_seqs, lay.block_size = b, u, ms, ps
        ops.decode_step_setup(hs, self._step_dev, lay, self._bt, self.seq_lens, slots,
                              self._plan_indices_gpu, stream_handle=sh)
        self._host_image_sent()
        if u:
            self._bt_pending.clear()
        # The whole page-index buffer goes to the decode (its pages are bounded
        # by the plan), so the launch does not change with the page count.
        w._install(sched, plan_v, indptr_v, lpl_v, self._plan_indices_gpu, self.num_heads,
                   self.num_kv_heads, self.head_dim, ps)
        lens_all[ids] += 1
        self._step_slots = step_slots
        return slots

    # ------------------------------------------------- step-buffer streams
    def _claim_step_buffer(self) -> int:
        """Order the current stream after every other stream that used the
        step buffer since its last upload, before it is rewritten; return the
        current stream's handle, now the step's stream.  (Stream objects are
        only made on the rare path where another stream was involved.)"""
        sh = _lib.current_stream_handle(self.device)
        if self._step_users:
            cur = torch.cuda.current_stream(self.device)
            for h, st in self._step_users.items():
                if h != sh:
                    cur.wait_stream(st)
            self._step_users = {}
        self._step_handle = sh
        self._step_stream_obj = None
        return sh

    def _step_stream_for_call(self) -> int:
        """Handle of the current stream for a launch that reads the step
        buffer.  A stream other than the step's is first ordered after the
        upload (eager calls only; under graph capture ordering is the
        caller's) and remembered, so that the next upload waits for it."""
        sh = _lib.current_stream_handle(self.device)
        if sh != self._step_handle and self._step_handle is not None \
                and sh not in self._step_users:
            if torch.cuda.is_current_stream_capturing():
                return sh
            cur = torch.cuda.current_stream(self.device)
            if self._step_stream_obj is None:
                self._step_stream_obj = torch.cuda.ExternalStream(self._step_handle,
                                                                  device=self.device)
            cur.wait_stream(self._step_stream_obj)
            self._step_users[sh] = cur
            if self._mixed_step_buf is not None:
                # a mixed step's buffer is freed at the next plan: keep the
                # allocator from reusing it before this stream ran
                self._mixed_step_buf.record_stream(cur)
        return sh

    def decode_graph_key(self) -> tuple:
        """What a decode launch of the current step bakes in besides its
        tensors: the device address of the step's plan and the launch shape of
        its schedule.  A graph that captured ``append_and_decode`` /
        ``decode`` calls after ``prepare_decode_step`` can be replayed after
        later ``prepare_decode_step`` calls while this key stays the same (the
        kernels read the new plan, lengths and page ids from the same
        buffers); when it changes, capture again and drop the old graph: its
        launches address a step buffer that may have been freed.  An empty
        key means the current plan is not a decode step's."""
        w = self._decode_wrapper
        s = w.schedule
        if (s is None or self._step_dev is None or self._step_slots is None
                or w._plan_dev.data_ptr() != self._step_dev.data_ptr()):
            return ()   # no decode step set up (or a mixed step's plan is current)
        # Without the fused append, append_and_decode's separate append reads
        # the step's slot tensor, a new allocation every step.
        slots = 0 if w.fused_append_supported else self._step_slots.data_ptr()
        return (self._step_dev.data_ptr(), w._indices.data_ptr(), w._num_indices, slots,
                s.batch, s.small_batch, s.num_segments,
                s.num_head_groups, s.heads_per_group, s.max_partitions, s.num_empty > 0,
                s.pieces_offset, s.nparts_offset, s.append_pieces)

    def prepare_step(self, decode_seq_ids: Sequence[int] = (),
                     prefill_seq_ids: Sequence[int] = (), prefill_lens: Sequence[int] = (),
                     continuation_seq_ids: Sequence[int] = (),
                     continuation_lens: Sequence[int] = (),
                     graph_n: Optional[int] = None) -> torch.Tensor:
        """Setup of a mixed step, the engine's ``step()`` (moe_engine.py:2555-2742,
        piecewise setup :3475-3556, continuation plan :3649-3728), with one
        host-to-device copy of all its metadata.

        Tokens are laid out ``[decode | new prefill | continuation]``: one per
        decode request (at its current length), ``prefill_lens[i]`` from
        position 0 for each new prompt (its length must be 0), and
        ``continuation_lens[i]`` from each continuation's current length.  The
        returned slot mapping (int64, padded with -1 to ``graph_n`` tokens)
        serves ``append`` of the step's K/V.  Afterwards the lengths are
        decode + 1, prompt length and offset + chunk; the decode wrapper is
        planned over the decode requests (``decode``: q rows in
        ``decode_seq_ids`` order) and the prefill wrapper over the
        continuations (``prefill``: their q rows, chunk after chunk).  New
        prompts attend over their own contiguous K/V outside the paged cache,
        as in the engine.  Pages must already cover every new token."""
        self._require_gpu()
        dec = [int(s) for s in decode_seq_ids]
        pre = [int(s) for s in prefill_seq_ids]
        con = [int(s) for s in continuation_seq_ids]
        plen = [int(n) for n in prefill_lens]
        clen = [int(n) for n in continuation_lens]
        if len(plen) != len(pre) or len(clen) != len(con):
            raise ValueError("one length per prefill / continuation sequence")
        if any(n <= 0 for n in plen + clen):
            raise ValueError("prefill and continuation lengths must be positive")
        D, P, C = len(dec), len(pre), len(con)
        ids = self._check_seq_ids(dec + pre + con)
        R = len(ids)
        counts = np.array([1] * D + plen + clen, dtype=np.int64)
        n_tok = int(counts.sum())
        graph_n = n_tok if graph_n is None else int(graph_n)
        if graph_n < n_tok:
            raise ValueError(f"graph_n ({graph_n}) is smaller than the step's {n_tok} tokens")
        self._step_slots = None
        if R == 0:
            return torch.full((graph_n,), -1, dtype=torch.int64, device=self.device)
        self._sync_seqs(ids.tolist())
        lens_all = self._seq_lens_cpu.numpy()
        ms, ps = self.max_seqs, self.page_size
        before = lens_all[ids].astype(np.int64)
        if P and (before[D:D + P] != 0).any():
            raise RuntimeError("a new prefill's sequence must be empty (free_seq it first)")
        after = before + counts
        if int(after.max()) > self.max_pages_per_seq * ps:
            raise RuntimeError(f"a sequence would exceed max_seq_len ({self.max_pages_per_seq * ps})")
        if self._dynamic_pages:
            short = [int(s) for s, n in zip(ids, after) if self._pool.seq_pages(int(s)) * ps < n]
            if short:
                raise RuntimeError(f"sequences {short} have no page for their new tokens "
                                   "(ensure_pages first)")
        d_after, c_after = after[:D], after[D + P:]

        def indptr_lpl(lens):
            ip = np.zeros(len(lens) + 1, np.int32)
            np.cumsum((lens + ps - 1) // ps, out=ip[1:])
            lpl = lens % ps
            return ip, np.where((lpl == 0) & (lens != 0), ps, lpl).astype(np.int32)

        # One pinned int32 image:
        #   ids[R] | qsl[R+1] | lens_before[ms] | lens_after[ms]
        #   | decode kv_indptr[D+1] | decode last_page_len[D]
        #   | continuation qo_indptr[C+1] | kv_indptr[C+1] | last_page_len[C]
        #   | block-table positions (int64) | page ids
        #   | decode schedule | prefill schedule (16-byte aligned each)
        pend = self._peek_bt_pending()
        u = 0 if pend is None else len(pend[0])
        dw, pw = self._decode_wrapper, self._prefill_wrapper
        o_qsl = R
        o_lb = o_qsl + R + 1
        o_la = o_lb + ms
        o_dip = o_la + ms
        o_dlpl = o_dip + D + 1
        o_cqo = o_dlpl + D
        o_cip = o_cqo + C + 1
        o_clpl = o_cip + C + 1
        o_pos = (o_clpl + C + 1) // 2 * 2
        o_val = o_pos + 2 * u
        o_dplan = (o_val + u + 3) // 4 * 4
        group = self.num_heads // self.num_kv_heads
        pcap = pw._plan_capacity(np.asarray(clen), group, self.num_kv_heads) if C else 0
        dcap = dw._plan_capacity(D) if D else 0
        while True:
            o_pplan = o_dplan + dcap
            hs = self._host_image(o_pplan + pcap)
            h = hs.numpy()
            h[:R] = ids
            h[o_qsl] = 0
            np.cumsum(counts, out=h[o_qsl + 1:o_lb])
            h[o_lb:o_la] = lens_all
            h[o_la:o_dip] = lens_all
            h[o_la + ids] = after
            dip, dlpl = indptr_lpl(d_after)
            h[o_dip:o_dlpl] = dip
            h[o_dlpl:o_cqo] = dlpl
            h[o_cqo] = 0
            np.cumsum(np.asarray(clen, np.int64), out=h[o_cqo + 1:o_cip])
            cip, clpl = indptr_lpl(c_after)
            h[o_cip:o_clpl] = cip
            h[o_clpl:o_clpl + C] = clpl
            if u:
                h[o_pos:o_pos + 2 * u].view(np.int64)[:] = pend[0]
                h[o_val:o_val + u] = pend[1]
            dsched = None
            if D:
                dsched = dw._schedule_into(h[o_dip:o_dlpl], h[o_dlpl:o_cqo], D, self.num_heads,
                                           self.num_kv_heads, self.head_dim, ps,
                                           hs[o_dplan:o_pplan])
                if dsched.plan_ints > dcap:
                    dcap = (dsched.plan_ints + 3) // 4 * 4
                    continue
            break
        psched = None
        if C:
            psched = pw._schedule_into(h[o_cqo:o_cip], h[o_cip:o_clpl], h[o_clpl:o_clpl + C], C,
                                       self.num_heads, self.num_kv_heads, self.head_dim, ps,
                                       True, hs[o_pplan:])
        self._check_page_counts(np.concatenate([(d_after + ps - 1) // ps,
                                                (c_after + ps - 1) // ps]))

        # The step's one upload; the plans' unused capacity is not sent.
        self._claim_step_buffer()
        dm = torch.empty(hs.numel(), dtype=torch.int32, device=self.device)
        self._mixed_step_buf = dm
        ops.stage_from_host(hs, dm, o_dplan + (int(dsched.plan_ints) if D else 0),
                            o_pplan, o_pplan + (int(psched.plan_ints) if C else 0))
        self._host_image_sent()
        if u:
            self._bt.view(-1).scatter_(0, dm[o_pos:o_val].view(torch.int64), dm[o_val:o_val + u])
            self._bt_pending.clear()
        ids_d = dm[:R]
        slots = torch.empty(graph_n, dtype=torch.int64, device=self.device)
        ops.compute_slot_mapping(self._bt, ids_d, dm[o_qsl:o_lb], dm[o_lb:o_la], n_tok, slots,
                                 block_size=ps)
        self.seq_lens.copy_(dm[o_la:o_dip])
        # A wrapper with no requests this step keeps no plan: a run() would
        # otherwise attend with the previous step's.
        if not D:
            dw._sched = None
        if not C:
            pw._sched = None
        if D:
            total = int(dip[-1])
            ops.copy_page_indices(self._bt, dm[o_dip:o_dlpl], self._plan_indices_gpu,
                                  seq_ids=ids_d[:D])
            dw._install(dsched, dm[o_dplan:o_dplan + dcap], dm[o_dip:o_dlpl],
                        dm[o_dlpl:o_cqo], self._plan_indices_gpu[:total], self.num_heads,
                        self.num_kv_heads, self.head_dim, ps)
        if C:
            total = int(cip[-1])
            ops.copy_page_indices(self._bt, dm[o_cip:o_clpl], self._prefill_indices_gpu,
                                  seq_ids=ids_d[D + P:])
            pw._install(psched, dm[o_pplan:o_pplan + max(pcap, 8)],
                        self._prefill_indices_gpu[:max(total, 1)], int(sum(clen)),
                        self.num_heads, self.num_kv_heads, self.head_dim, ps)
        lens_all[ids] = after
        return slots

    # ------------------------------------------------------- per-layer ops
    def append(self, layer: int, key: torch.Tensor, value: torch.Tensor,
               slot_mapping: torch.Tensor) -> None:
        ops.reshape_and_cache_flash(key, value, self.k_cache[layer], self.v_cache[layer],
                                    slot_mapping, "auto")

    def append_and_decode(self, layer: int, key: torch.Tensor, value: torch.Tensor,
                          q: torch.Tensor, out: Optional[torch.Tensor] = None,
                          return_lse: bool = False):
        """``append(layer, key, value, slots)`` then ``decode(layer, q)`` for
        the step set up by the last ``prepare_decode_step``: one launch when
        the decode wrapper supports the fused append, else the two calls.
        ``key``/``value`` are the step's new rows ``[B, Hkv, D]`` in the order
        of that call's ``seq_ids``; the result is the same either way, bit for
        bit."""
        slots = self._step_slots
        if slots is None:
            self._require_gpu()
            raise RuntimeError("append_and_decode needs a prepare_decode_step first")
        w = self._decode_wrapper
        sh = self._step_stream_for_call()
        kv = self._layer_kv[layer]
        if w._fused_ok:
            return w._launch(q, None, out, None, return_lse, sh, key, value, kv)
        self.append(layer, key, value, slots)
        return w._launch(q, None, out, None, return_lse, sh, None, None, kv)

    def decode(self, layer: int, q: torch.Tensor, out: Optional[torch.Tensor] = None,
               return_lse: bool = False):
        """Decode attention of the planned requests over ``layer`` (the
        engine's FlashInfer run, moe_engine.py:3907-3909)."""
        self._require_gpu()
        return self._decode_wrapper._launch(q, None, out, None, return_lse,
                                            self._step_stream_for_call(), None, None,
                                            self._layer_kv[layer])

    def gather(self, layer: int, seq_ids: Sequence[int], out_key: Optional[torch.Tensor] = None,
               out_value: Optional[torch.Tensor] = None):
        """Contiguous ``[sum(len), heads, dim]`` K and V of the given sequences
        (their current ``seq_lens``), in order."""
        self._require_gpu()
        ids = self._check_seq_ids(seq_ids)
        self._sync_seqs(seq_ids)
        lens = self._seq_lens_cpu.numpy()[ids].astype(np.int32)
        cu = np.zeros(len(ids) + 1, dtype=np.int32)
        np.cumsum(lens, out=cu[1:])
        total = int(cu[-1])
        for name, t in (("out_key", out_key), ("out_value", out_value)):
            if t is not None and (t.dim() < 1 or t.shape[0] < total):
                raise RuntimeError(f"{name} holds {t.shape[0] if t.dim() else 0} rows; "
                                   f"the sequences have {total} tokens")
        cu_t = self._to_device(cu)
        rows = self.block_table.index_select(0, self._to_device(ids))
        if out_key is None:
            out_key = torch.empty(total, self.num_kv_heads, self.head_dim, dtype=self.dtype,
                                  device=self.device)
        if out_value is None:
            out_value = torch.empty(total, self.num_kv_heads, self.head_dim, dtype=self.dtype,
                                    device=self.device)
        return ops.gather_kv(self.k_cache[layer], self.v_cache[layer], rows, cu_t,
                             int(lens.max()) if len(lens) else 0, out_key, out_value)

    # ----------------------------------------------------------------- swap
    def _side_stream(self) -> torch.cuda.Stream:
        """Stream of the swap's gather / scatter kernels."""
        if self._swap_stream is None:
            self._swap_stream = torch.cuda.Stream(device=self.device)
        return self._swap_stream

    def _dma_stream(self) -> torch.cuda.Stream:
        """Stream of the swap's host-link copies."""
        if self._copy_stream is None:
            self._copy_stream = torch.cuda.Stream(device=self.device)
        return self._copy_stream

    # The pinned step images form a ring of _META_RING slots, one per step.
    # A slot is rewritten only after the kernel that read it last (R steps
    # ago) has run.  Recording an event costs the host ~4 us, so one is
    # recorded every _META_EVERY steps: before step t reuses its slot, the
    # host waits for the first event recorded at or after step t - R, which
    # exists (R >= _META_EVERY) and was recorded before step t.  Every step's
    # upload runs after the previous steps' (each setup orders its stream
    # after the streams that used the step buffer), so that event's
    # completion covers step t - R.
    _META_RING = 8
    _META_EVERY = 4

    def _meta_slot(self, n: int) -> list:
        t = self._meta_step
        slot = self._meta_ring[t % self._META_RING]
        if t >= self._META_RING:
            need = t - self._META_RING
            ev = self._meta_events
            while ev and ev[0][0] < need:
                ev.popleft()
            if ev and ev[0][0] < t:
                ev[0][1].synchronize()
        if slot[0] is None or slot[0].numel() < n:
            slot[0] = torch.empty(max(n, 2 * (0 if slot[0] is None else slot[0].numel())),
                                  dtype=torch.int32, pin_memory=True)
            slot[1] = slot[0].numpy()
        return slot

    def _host_image(self, n: int) -> torch.Tensor:
        """A pinned int32 image of ``n`` entries for the step's metadata: the
        ring's next slot, once the upload that last read it has run."""
        return self._meta_slot(n)[0][:n]

    def _host_image_np(self, n: int):
        """``_host_image`` for the decode step: the ring slot's whole pinned
        tensor (its first ``n`` entries are the image) and a numpy view of
        those ``n`` entries (no per-step tensor view)."""
        slot = self._meta_slot(n)
        return slot[0], slot[1][:n]

    def _host_image_sent(self) -> None:
        """Mark the slot ``_host_image`` returned as read by the upload just
        issued on the current stream, and move to the next slot."""
        t = self._meta_step
        if t % self._META_EVERY == 0:
            e = torch.cuda.Event()
            e.record()
            self._meta_events.append((t, e))
        self._meta_step = t + 1

    def _staging_buf(self) -> torch.Tensor:
        if self._staging is None:
            self._staging = torch.empty(self._staging_bytes, dtype=torch.uint8, device=self.device)
        return self._staging

    # Round trips of the swap warm-up: at least a large eviction's chunk count
    # (an 8.6 GB swap through 256 MiB staging halves makes 32 copies).
    _SWAP_WARM_COPIES = 32
    _SWAP_WARM_BYTES = 16 << 20

    def reserve_swap(self) -> None:
        """Allocate the swap staging buffer and create the side and DMA
        streams now, so that the first ``swap_out`` does not pay for them on
        the engine loop (a 512 MiB device allocation and two stream creations
        take ~17 ms of host time).  Without this call they are made on the
        first swap.

        The first call also warms the runtime's copy path: 32 round trips of
        a 16 MiB pinned buffer through the staging on the DMA stream, ordered
        by events as a swap's chunks are, and a gather of block 0 of every
        layer into the staging on the side stream (it reads the caches and
        writes only the staging).  A process's first few dozen such copies
        and stream waits cost the host far more than later ones: the first
        8.6 GB swap-out (32 chunks) took 18-31 ms to enqueue without the
        warm-up and 3 ms after it; copies of 64 KB, or fewer round trips,
        left 5-15 ms.  The warm-up takes ~25 ms and waits for it to finish."""
        self._require_gpu()
        st = self._staging_buf()
        side, dma = self._side_stream(), self._dma_stream()
        if self._swap_warm:
            return
        # Work already enqueued on the current stream (which the staging's
        # memory may still serve) and earlier swaps' staging use (kernels on
        # one stream, copies on the other) finish before the warm-up
        # overwrites the staging.
        side.wait_stream(torch.cuda.current_stream(self.device))
        side.wait_stream(dma)
        dma.wait_stream(side)
        nb = min(self._SWAP_WARM_BYTES, st.numel())
        host = hostmem.pinned_empty(nb, self.device)
        for _ in range(self._SWAP_WARM_COPIES):
            e = torch.cuda.Event()
            e.record(side)
            dma.wait_event(e)
            with torch.cuda.stream(dma):
                host.copy_(st[:nb], non_blocking=True)
            e = torch.cuda.Event()
            e.record(dma)
            side.wait_event(e)
            with torch.cuda.stream(dma):
                st[:nb].copy_(host, non_blocking=True)
            e = torch.cuda.Event()
            e.record(dma)
            side.wait_event(e)
        per = 2 * ops.block_bytes(self.k_cache[0])
        if per <= st.numel():
            with torch.cuda.stream(side):
                ids0 = torch.zeros(1, dtype=torch.int32, device=self.device)
            for layer in range(self.num_layers):
                ops.gather_blocks(self.k_cache[layer], self.v_cache[layer], ids0, st[:per],
                                  stream=side)
        side.synchronize()
        dma.synchronize()
        self._swap_warm = True

    def _staging_halves(self, per_block: int):
        """The staging buffer as two halves and the blocks one half holds."""
        st = self._staging_buf()
        half = st.numel() // 2 // 256 * 256
        if half < per_block:
            raise RuntimeError(f"staging of {st.numel()} bytes cannot hold two blocks of "
                               f"{per_block} bytes")
        return (st[:half], st[half:2 * half]), half // per_block

    def _pipelined_swap(self, to_host: bool, ids_t: torch.Tensor, n: int,
                        host: torch.Tensor):
        """Move blocks ``ids_t`` of every layer between the caches and
        ``host`` ([layers][n][2][block_bytes]) through the two staging halves:
        gather/scatter kernels on the side stream, the host-link copies on the
        DMA stream, ordered by events, so that the copy of one chunk overlaps
        the kernels of the next.  A chunk fills a staging half with consecutive
        (layer, block) items of the host image, across layer boundaries (one
        kernel per layer it touches, one copy), so small swaps make few large
        copies: each copy costs the DMA queue a fixed ~0.1-0.5 ms.  A half is
        reused only after its previous copy (swap-out) or scatter (swap-in)
        completed.  Returns (start, end) events; the side stream has already
        waited for the current stream."""
        side, dma = self._side_stream(), self._dma_stream()
        bb = ops.block_bytes(self.k_cache[0])
        per = 2 * bb
        halves, chunk = self._staging_halves(per)
        start = torch.cuda.Event(enable_timing=True)
        (side if to_host else dma).record_event(start)
        if not to_host:
            dma.wait_event(start)
        end = None
        total = self.num_layers * n
        for i, f0 in enumerate(range(0, total, chunk)):
            c = min(chunk, total - f0)
            b = i % 2
            buf = halves[b][: c * per]
            hview = host[f0 * per: (f0 + c) * per]
            # (layer, first block, end block, offset in the chunk) per layer touched
            segs = []
            f = f0
            while f < f0 + c:
                layer, j0 = divmod(f, n)
                j1 = min(n, j0 + (f0 + c - f))
                segs.append((layer, j0, j1, f - f0))
                f += j1 - j0
            done = torch.cuda.Event(enable_timing=True)
            if to_host:
                if self._staging_free[b] is not None:
                    side.wait_event(self._staging_free[b])
                for layer, j0, j1, o in segs:
                    ops.gather_blocks(self.k_cache[layer], self.v_cache[layer], ids_t[j0:j1],
                                      buf[o * per: (o + j1 - j0) * per], stream=side)
                gathered = torch.cuda.Event()
                gathered.record(side)
                dma.wait_event(gathered)
                with torch.cuda.stream(dma):
                    hview.copy_(buf, non_blocking=True)
                done.record(dma)
            else:
                if self._staging_free[b] is not None:
                    dma.wait_event(self._staging_free[b])
                with torch.cuda.stream(dma):
                    buf.copy_(hview, non_blocking=True)
                loaded = torch.cuda.Event()
                loaded.record(dma)
                side.wait_event(loaded)
                for layer, j0, j1, o in segs:
                    ops.scatter_blocks(buf[o * per: (o + j1 - j0) * per], ids_t[j0:j1],
                                       self.k_cache[layer], self.v_cache[layer], stream=side)
                done.record(side)
            self._staging_free[b] = done
            end = done
        ids_t.record_stream(side)
        if end is None:
            end = torch.cuda.Event(enable_timing=True)
            end.record(side)
        # Both streams may still be running: make the side stream (which the
        # callers wait on) finish after the last copy too.
        side.wait_event(end)
        last = torch.cuda.Event(enable_timing=True)
        last.record(side)
        return start, last

    def _reclaim(self, need: int = 0) -> None:
        """Return pages of finished swap-outs to the free list; block on the
        oldest pending swap-out only if the pool cannot serve ``need`` pages."""
        self._swaps.reclaim(self._pool, need)

    def synchronize_swaps(self) -> None:
        for st in (self._swap_stream, self._copy_stream):
            if st is not None:
                st.synchronize()
        if self._dynamic_pages:
            self._reclaim(need=self.total_pages + 1)

    def swap_out(self, seq_ids: Sequence[int], host: Optional[torch.Tensor] = None) -> SwapHandle:
        """Evict whole sequences to pinned host memory on the side stream.

        The sequences stop being resident (pages detached, block-table rows
        -1, length 0); their pages rejoin the free list once the copy is done.
        The side stream first waits for all work already enqueued on the
        current stream, so earlier appends are included.  ``host`` may be a
        caller-allocated pinned uint8 buffer of at least
        ``layers * pages * 2 * block_bytes`` bytes (otherwise one is
        allocated)."""
        self._require_gpu()
        self._require_dynamic()
        seq_ids = [int(s) for s in seq_ids]
        cur = torch.cuda.current_stream(self.device)
        self._sync_seqs(seq_ids)
        lens, npages, ids = [], [], []
        for sid in seq_ids:
            pages = self._pool.detach(sid)
            lens.append(int(self._seq_lens_cpu[sid]))
            npages.append(len(pages))
            ids.extend(pages)
            if pages:
                self._bt_write(sid, 0, [-1] * len(pages))
            self._seq_lens_cpu[sid] = 0
        self._lens_to_device()
        n = len(ids)
        bb = ops.block_bytes(self.k_cache[0])
        nbytes = self.num_layers * n * 2 * bb
        if host is None:
            host = hostmem.pinned_empty(nbytes, self.device)
        elif host.is_cuda or not host.is_pinned() or host.numel() * host.element_size() < nbytes:
            raise RuntimeError(f"host buffer must be pinned CPU memory of >= {nbytes} bytes")
        ids_t = self._to_device(np.asarray(ids, dtype=np.int32))
        self._side_stream().wait_stream(cur)
        start, ev = self._pipelined_swap(True, ids_t, n, host)
        # The host buffer must outlive the D2H copy even if the handle is dropped.
        self._swaps.add_swap_out(ev, ids, [ids_t, host])
        return SwapHandle(seq_ids, lens, npages, ids_t, host, ev, out_start=start, num_bytes=nbytes)

    def swap_in(self, handle: SwapHandle, wait: bool = False,
                seq_ids: Optional[Sequence[int]] = None) -> None:
        """Restore an evicted handle into freshly allocated pages.

        Allocation and block-table updates happen now; the H2D copies and the
        scatter run on the side stream after everything already enqueued on
        the current stream.  Later ``plan_decode`` / ``gather`` / ``swap_out``
        of these sequences make the current stream wait for the restore;
        ``wait=True`` does so immediately.  ``seq_ids`` restores into other
        (non-resident) sequence slots, one per evicted sequence, in order --
        a preempted request may resume in whatever slot is free."""
        self._require_gpu()
        self._require_dynamic()
        if handle.restored:
            raise RuntimeError("swap handle already restored")
        targets = list(handle.seq_ids) if seq_ids is None else [int(s) for s in seq_ids]
        if len(targets) != len(handle.seq_ids) or len(set(targets)) != len(targets):
            raise ValueError("seq_ids must name one distinct slot per evicted sequence")
        cur = torch.cuda.current_stream(self.device)
        dst = []
        for sid, n, ln in zip(targets, handle.num_pages, handle.seq_lens):
            if self._pool.seq_pages(sid) != 0 or int(self._seq_lens_cpu[sid]) != 0:
                raise RuntimeError(f"seq {sid} is resident; free it before swap_in")
            self.alloc_pages(sid, n)
            dst.extend(self._pool.seq_page_list[sid])
            self._seq_lens_cpu[sid] = ln
        self._lens_to_device()
        dst_t = self._to_device(np.asarray(dst, dtype=np.int32))
        side = self._side_stream()
        side.wait_stream(cur)
        side.wait_event(handle.out_event)
        self._dma_stream().wait_stream(side)
        start, ev = self._pipelined_swap(False, dst_t, len(dst), handle.host)
        handle.in_start = start
        self._swaps.add_swap_in(ev, targets, [dst_t, handle.host])
        handle.in_event = ev
        handle.dst_block_ids = dst_t
        handle.restored = True
        handle.seq_ids = targets
        if wait:
            self._sync_seqs(targets)
