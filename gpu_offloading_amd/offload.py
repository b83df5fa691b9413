"""KV offload to pinned host memory, as end-to-end policies.

Two users of the host link, both built on this package's copy paths:

* ``SwapPreemption`` -- preemption by swapping.  The reference scheduler
  preempts by recompute (src/MoE/scheduler.py:315-378): the LIFO victim's
  pages are freed and its whole prompt + output is prefilled again later.
  Here the victim's KV is evicted with ``PagedKVCache.swap_out`` (gather to
  HBM staging + D2H on side streams, pages returned once the copy is done)
  and restored with ``swap_in`` when the request is admitted again, into
  whatever slot is free, so it resumes decoding with no recompute.

* ``PagedOffloadKV`` + ``KVOffloadPipeline`` -- the dense sandbox's
  layer-wise KV offload (src/dense/include/paged_offload_transformer.py):
  x-packed heap, layer 0 resident, and for layers 1.. a fixed share of every
  sequence's blocks kept in pinned host memory and staged per layer into one
  of two GPU scratchpads (layer parity) by a host-to-device stream, while the
  newly written prefill blocks of the scratchpad go back by a device-to-host
  stream.  Unlike the reference's timing harness (whose compute stream waits
  on events the copy streams record only later in program order), every
  wait here refers to an event already enqueued, so the staged history is
  the one attention reads:
    H2D(l) [decode region of scratchpad l%2] waits compute_done of the
      previous layer on that scratchpad;
    append(l) [writes the prefill region] waits D2H of that previous layer;
    decode attention(l) waits H2D(l);
    D2H(l) [prefill region -> host] waits the layer's prefill.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence

import numpy as np
import torch

from . import hostmem
from .kv_cache import PagedKVCache, SwapHandle

__all__ = ["SwapPreemption", "PagedOffloadKV", "KVOffloadPipeline"]


# --------------------------------------------------------------------------
# Preemption by swap
# --------------------------------------------------------------------------
class SwapPreemption:
    """Swap-instead-of-recompute preemption over a dynamic ``PagedKVCache``.

    The scheduler calls ``preempt(slot, key)`` where the reference resets the
    victim for recompute (scheduler.py:329-352): the request keeps its
    ``seq_len`` / ``num_computed_tokens`` and its KV goes to host memory.  At
    admission, ``pages_to_resume(key)`` is the page demand and
    ``resume(key, slot)`` restores the KV into the given free slot.  The
    victim's pages return to the free list as soon as its D2H copy has run
    (``PagedKVCache`` reclaims them lazily, or on demand when an allocation
    needs them).
    """

    def __init__(self, cache: PagedKVCache, host_budget_bytes: Optional[int] = None):
        self.cache = cache
        self.host_budget_bytes = host_budget_bytes
        self._swapped: Dict[object, SwapHandle] = {}
        self.swaps_out = 0
        self.swaps_in = 0

    @property
    def host_bytes_in_use(self) -> int:
        return sum(h.bytes_per_direction for h in self._swapped.values())

    def can_preempt(self, slot: int) -> bool:
        """Whether the victim's KV fits the host budget."""
        if self.host_budget_bytes is None:
            return True
        need = self.cache.num_layers * self.cache.seq_pages(slot) * 2 * \
            self.cache.k_cache[0][0].numel() * self.cache.k_cache[0].element_size()
        return self.host_bytes_in_use + need <= self.host_budget_bytes

    def preempt(self, slot: int, key, host=None) -> SwapHandle:
        """Swap ``slot`` out under ``key``.  ``host``: an optional pinned host
        buffer to hold the image (``PagedKVCache.swap_out``); an engine that
        keeps a pool of them avoids pinning a new buffer per preemption."""
        if key in self._swapped:
            raise RuntimeError(f"request {key!r} is already swapped out")
        handle = self.cache.swap_out([slot], host=host)
        self._swapped[key] = handle
        self.swaps_out += 1
        return handle

    def is_swapped(self, key) -> bool:
        return key in self._swapped

    def swapped_len(self, key) -> int:
        return self._swapped[key].seq_lens[0]

    def pages_to_resume(self, key) -> int:
        return self._swapped[key].num_pages[0]

    def resume(self, key, slot: int, wait: bool = False) -> int:
        """Restore ``key`` into ``slot``; returns its sequence length."""
        handle = self._swapped.pop(key)
        self.cache.swap_in(handle, wait=wait, seq_ids=[slot])
        self.swaps_in += 1
        return handle.seq_lens[0]

    def drop(self, key) -> None:
        """Forget a swapped request (finished or switched to recompute); its
        host buffer is released once no copy uses it."""
        self._swapped.pop(key, None)


# --------------------------------------------------------------------------
# Layer-wise KV offload (dense sandbox)
# --------------------------------------------------------------------------
class PagedOffloadKV:
    """KV state of the dense sandbox's offload mode
    (paged_offload_transformer.py:12-300), x-packed layout.

    Mixed batch: prefill sequences first (whole prompt this step), then decode
    sequences (history + 1 new token).  Per sequence of ``tb`` blocks,
    ``int(tb * kv_offload_ratio)`` leading blocks are offloaded in layers
    1..L-1.  Heap = layer 0 (all blocks) + layers 1.. (resident blocks) + two
    scratchpads of the batch's offloaded blocks, each ``[decode region |
    prefill region]`` in sequence order.  ``block_tables[l][b]`` lists the
    scratchpad ids (parity l % 2) first, then resident ids.  Pinned host
    buffers hold, per offloaded layer, the decode sequences' offloaded
    history (read each step) and the prefill sequences' offloaded blocks
    (written each step).
    """

    def __init__(self, decode_lengths: Sequence[int], prefill_lengths: Sequence[int],
                 num_layers: int, num_heads: int, head_dim: int, kv_offload_ratio: float,
                 block_size: int = 16, dtype: torch.dtype = torch.float16,
                 device: str | torch.device = "cuda", allocation_mode: str = "contiguous",
                 seed: int = 0):
        if block_size != 16 or head_dim != 128:
            raise ValueError("the x-packed kernels take block_size 16 and head_dim 128")
        if not 0.0 <= kv_offload_ratio <= 1.0:
            raise ValueError("kv_offload_ratio must be in [0, 1]")
        if num_layers < 1:
            raise ValueError("num_layers must be >= 1")
        self.num_layers, self.num_heads, self.head_dim = num_layers, num_heads, head_dim
        self.block_size, self.dtype, self.device = block_size, dtype, torch.device(device)
        self.x = 16 // torch.tensor([], dtype=dtype).element_size()
        self.decode_lengths = [int(v) for v in decode_lengths]
        self.prefill_lengths = [int(v) for v in prefill_lengths]
        self.num_prefills, self.num_decodes = len(self.prefill_lengths), len(self.decode_lengths)
        self.batch_size = self.num_prefills + self.num_decodes
        self.num_prefill_tokens = sum(self.prefill_lengths)
        self.total_tokens = self.num_prefill_tokens + self.num_decodes

        bs = block_size
        blocks = [math.ceil(n / bs) for n in self.prefill_lengths] + \
                 [math.ceil((n + 1) / bs) for n in self.decode_lengths]
        self.blocks_per_seq = blocks
        self.offload_counts = [int(tb * kv_offload_ratio) for tb in blocks]
        self.resident_counts = [tb - o for tb, o in zip(blocks, self.offload_counts)]
        P = self.num_prefills
        self.prefill_offload_blocks = sum(self.offload_counts[:P])
        self.decode_offload_blocks = sum(self.offload_counts[P:])
        off = self.prefill_offload_blocks + self.decode_offload_blocks
        self.offload_blocks = off
        res_pool = sum(blocks) + sum(self.resident_counts) * (num_layers - 1)
        heap = res_pool + 2 * off
        self.heap_blocks = heap
        self.scratchpad_ranges = [(heap - 2 * off, heap - off), (heap - off, heap)]

        h, d, x = num_heads, head_dim, self.x
        self.key_heap = torch.zeros(heap, h, d // x, bs, x, dtype=dtype, device=self.device)
        self.val_heap = torch.zeros(heap, h, d, bs, dtype=dtype, device=self.device)
        dec_off, pre_off = self.decode_offload_blocks, self.prefill_offload_blocks

        def pinned(n, shape):
            if self.device.type != "cuda":
                return torch.zeros((n,) + shape, dtype=dtype)
            numel = n * math.prod(shape)
            t = hostmem.pinned_empty(numel * dtype.itemsize,
                                     self.device, dtype)
            return t.zero_().view((n,) + shape)

        kshape, vshape = (h, d // x, bs, x), (h, d, bs)
        self.k_offload_cpu = [pinned(dec_off, kshape) for _ in range(num_layers - 1)]
        self.v_offload_cpu = [pinned(dec_off, vshape) for _ in range(num_layers - 1)]
        self.k_prefill_cpu = [pinned(pre_off, kshape) for _ in range(num_layers - 1)]
        self.v_prefill_cpu = [pinned(pre_off, vshape) for _ in range(num_layers - 1)]

        # sequence offsets inside a scratchpad: decode region, then prefill region
        sp_off, cur_dec, cur_pre = [], 0, dec_off
        for b in range(self.batch_size):
            if b < P:
                sp_off.append(cur_pre)
                cur_pre += self.offload_counts[b]
            else:
                sp_off.append(cur_dec)
                cur_dec += self.offload_counts[b]
        self.scratchpad_seq_offsets = sp_off
        if allocation_mode == "random":
            pool = torch.randperm(res_pool, generator=torch.Generator().manual_seed(seed))
        elif allocation_mode == "contiguous":
            pool = torch.arange(res_pool)
        else:
            raise ValueError("allocation_mode must be 'contiguous' or 'random'")
        pool = pool.to(torch.int32)
        maxb = max(blocks) if blocks else 0
        bt = torch.zeros(num_layers, self.batch_size, maxb, dtype=torch.int32)
        ptr = 0
        for b in range(self.batch_size):
            n_tot, n_off, n_res = blocks[b], self.offload_counts[b], self.resident_counts[b]
            bt[0, b, :n_tot] = pool[ptr:ptr + n_tot]
            ptr += n_tot
            for layer in range(1, num_layers):
                base = self.scratchpad_ranges[layer % 2][0] + sp_off[b]
                bt[layer, b, :n_off] = torch.arange(base, base + n_off, dtype=torch.int32)
                bt[layer, b, n_off:n_tot] = pool[ptr:ptr + n_res]
                ptr += n_res
        self.block_tables_cpu = bt
        self.block_tables = bt.to(self.device)

        # slot mapping: prefill tokens 0..len-1, then each decode's new token
        rows, pos = [], []
        for b, n in enumerate(self.prefill_lengths):
            rows += [b] * n
            pos += list(range(n))
        for i, n in enumerate(self.decode_lengths):
            rows.append(P + i)
            pos.append(n)
        rows_t, pos_t = torch.tensor(rows, dtype=torch.long), torch.tensor(pos, dtype=torch.long)
        sm = torch.empty(num_layers, len(rows), dtype=torch.long)
        for layer in range(num_layers):
            phys = bt[layer][rows_t, pos_t // bs].long() if rows else torch.empty(0, dtype=torch.long)
            sm[layer] = phys * bs + pos_t % bs
        self.slot_mapping = sm.to(self.device)
        self.decode_context_lens = torch.tensor([n + 1 for n in self.decode_lengths],
                                                dtype=torch.int32, device=self.device)
        max_len = max(self.prefill_lengths + [n + 1 for n in self.decode_lengths] + [1])
        self.max_decode_len = max([n + 1 for n in self.decode_lengths] + [1])
        parts = (max_len + 511) // 512
        nd = max(self.num_decodes, 1)
        self.exp_sums = torch.empty(nd, h, parts, dtype=torch.float32, device=self.device)
        self.max_logits = torch.empty_like(self.exp_sums)
        self.tmp_output = torch.empty(nd, h, parts, d, dtype=dtype, device=self.device)

    # ------------------------------------------------------------ helpers
    def decode_block_table(self, layer: int) -> torch.Tensor:
        return self.block_tables[layer, self.num_prefills:]

    def scratchpad_decode_blocks(self, layer: int) -> slice:
        s = self.scratchpad_ranges[layer % 2][0]
        return slice(s, s + self.decode_offload_blocks)

    def scratchpad_prefill_blocks(self, layer: int) -> slice:
        s, e = self.scratchpad_ranges[layer % 2]
        return slice(s + self.decode_offload_blocks, e)

    def _blocks(self, tokens: torch.Tensor, nblk: int, key: bool) -> torch.Tensor:
        """[n, H, D] tokens as x-packed blocks, zero-padded past n: K
        [nblk, H, D/x, bs, x] or V [nblk, H, D, bs]."""
        bs, h, d, x = self.block_size, self.num_heads, self.head_dim, self.x
        pad = torch.zeros(nblk * bs, h, d, dtype=self.dtype, device=self.device)
        pad[:tokens.shape[0]] = tokens.to(self.device, self.dtype)
        t = pad.view(nblk, bs, h, d)
        if key:
            return t.view(nblk, bs, h, d // x, x).permute(0, 2, 3, 1, 4).contiguous()
        return t.permute(0, 2, 3, 1).contiguous()

    def load_history(self, layer: int, decode_index: int, key: torch.Tensor,
                     value: torch.Tensor) -> None:
        """Place the ``decode_lengths[i]`` history tokens (``[n, H, D]``) of
        decode sequence i for ``layer`` where the layout keeps them: resident
        blocks in the heap, offloaded ones (layers >= 1) in the pinned host
        buffer that the pipeline stages each step."""
        b = self.num_prefills + decode_index
        n = self.decode_lengths[decode_index]
        if key.shape[0] != n or value.shape[0] != n:
            raise ValueError(f"history of decode {decode_index} has {n} tokens")
        nblk = self.blocks_per_seq[b]
        kb = self._blocks(key, nblk, True)
        vv = self._blocks(value, nblk, False)
        ids = self.block_tables_cpu[layer, b, :nblk].long()
        n_off = self.offload_counts[b] if layer > 0 else 0
        if n_off:
            o = self.scratchpad_seq_offsets[b]
            self.k_offload_cpu[layer - 1][o:o + n_off].copy_(kb[:n_off].cpu())
            self.v_offload_cpu[layer - 1][o:o + n_off].copy_(vv[:n_off].cpu())
        res = ids[n_off:].to(self.device)
        self.key_heap[res] = kb[n_off:]
        self.val_heap[res] = vv[n_off:]


class KVOffloadPipeline:
    """Three streams (compute = the current stream, host-to-device,
    device-to-host) staging ``PagedOffloadKV``'s offloaded blocks per layer
    (paged_offload_transformer.py:343-458, with the ordering described in
    this module's docstring).  Per step::

        pipe.begin_step()                 # history loads of layers 1 and 2
        for layer in range(L):
            pipe.before_append(layer)     # scratchpad's prefill region free
            ... reshape_and_cache(...)    # slot_mapping[layer]
            pipe.prefill_done(layer)      # D2H of the new prefill blocks
            pipe.before_decode(layer)     # history staged
            ... paged_attention_v2(...)   # decode_block_table(layer)
            pipe.layer_done(layer)        # scratchpad reusable: H2D(layer+2)
    """

    def __init__(self, kv: PagedOffloadKV):
        self.kv = kv
        self.h2d = torch.cuda.Stream(device=kv.device)
        self.d2h = torch.cuda.Stream(device=kv.device)
        self._last_compute: List[Optional[torch.cuda.Event]] = [None, None]
        self._last_d2h: List[Optional[torch.cuda.Event]] = [None, None]
        self._h2d_ready: Dict[int, torch.cuda.Event] = {}
        self.h2d_bytes = 0
        self.d2h_bytes = 0
        self._t: Dict[str, List[torch.cuda.Event]] = {"h2d": [], "d2h": []}

    def _cur(self) -> torch.cuda.Stream:
        return torch.cuda.current_stream(self.kv.device)

    def _enqueue_h2d(self, layer: int) -> None:
        kv, sp = self.kv, layer % 2
        ev = torch.cuda.Event()
        with torch.cuda.stream(self.h2d):
            if self._last_compute[sp] is not None:
                self.h2d.wait_event(self._last_compute[sp])
            if kv.decode_offload_blocks:
                t0 = torch.cuda.Event(enable_timing=True)
                t1 = torch.cuda.Event(enable_timing=True)
                t0.record(self.h2d)
                r = kv.scratchpad_decode_blocks(layer)
                kv.key_heap[r].copy_(kv.k_offload_cpu[layer - 1], non_blocking=True)
                kv.val_heap[r].copy_(kv.v_offload_cpu[layer - 1], non_blocking=True)
                t1.record(self.h2d)
                self._t["h2d"] += [t0, t1]
                self.h2d_bytes += (kv.k_offload_cpu[layer - 1].nbytes +
                                   kv.v_offload_cpu[layer - 1].nbytes)
            ev.record(self.h2d)
        self._h2d_ready[layer] = ev

    def begin_step(self) -> None:
        for layer in (1, 2):
            if layer < self.kv.num_layers:
                self._enqueue_h2d(layer)

    def before_append(self, layer: int) -> None:
        if layer >= 1 and self._last_d2h[layer % 2] is not None:
            self._cur().wait_event(self._last_d2h[layer % 2])

    def prefill_done(self, layer: int) -> None:
        kv = self.kv
        if layer < 1 or not kv.prefill_offload_blocks:
            return
        ready = torch.cuda.Event()
        ready.record(self._cur())
        done = torch.cuda.Event()
        with torch.cuda.stream(self.d2h):
            self.d2h.wait_event(ready)
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record(self.d2h)
            r = kv.scratchpad_prefill_blocks(layer)
            kv.k_prefill_cpu[layer - 1].copy_(kv.key_heap[r], non_blocking=True)
            kv.v_prefill_cpu[layer - 1].copy_(kv.val_heap[r], non_blocking=True)
            t1.record(self.d2h)
            self._t["d2h"] += [t0, t1]
            self.d2h_bytes += kv.k_prefill_cpu[layer - 1].nbytes + kv.v_prefill_cpu[layer - 1].nbytes
            done.record(self.d2h)
        self._last_d2h[layer % 2] = done

    def before_decode(self, layer: int) -> None:
        if layer >= 1:
            self._cur().wait_event(self._h2d_ready.pop(layer))

    def layer_done(self, layer: int) -> None:
        if layer < 1:
            return
        ev = torch.cuda.Event()
        ev.record(self._cur())
        self._last_compute[layer % 2] = ev
        if layer + 2 < self.kv.num_layers:
            self._enqueue_h2d(layer + 2)

    def synchronize(self) -> None:
        self.h2d.synchronize()
        self.d2h.synchronize()

    def copy_seconds(self) -> Dict[str, float]:
        """Summed stream time of the recorded H2D / D2H copies (after a
        synchronize); resets the record."""
        out = {}
        for k, evs in self._t.items():
            out[k] = sum(evs[i].elapsed_time(evs[i + 1]) for i in range(0, len(evs), 2)) * 1e-3
            evs.clear()
        return out
