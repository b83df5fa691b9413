"""Reference-shaped Python ops over libkvc.so (include/kvc.h).

Each op keeps the signature and error behaviour (``RuntimeError``) of the
library call the reference engine makes on this path, and launches a HIP
kernel on the current torch stream (or the stream given).  There is no CPU or
PyTorch fallback: without libkvc.so every op raises.

Reference call sites (aojsd/GPU_Offloading):
  reshape_and_cache_flash   src/MoE/moe_engine.py:2059-2062, :2344-2347
  merge_attention_states    src/dense/offload_kv_attn.py:24-39
  compute_slot_mapping      src/MoE/moe_engine.py:3514-3541 (eager :1308-1316)
  copy_page_indices         src/MoE/moe_engine.py:1937-1946
  stage_from_host           src/MoE/moe_engine.py:3493-3494, 3506-3507
  gather_kv / *_blocks / swap_*   new API (the engine has no gather or swap;
                            precedents moe_engine.py:4163-4183 and
                            src/dense/include/paged_offload_transformer.py:111-134, 394-418)
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import _lib

__all__ = [
    "reshape_and_cache_flash",
    "gather_kv",
    "merge_attention_states",
    "compute_slot_mapping",
    "copy_page_indices",
    "stage_from_host",
    "gather_blocks",
    "scatter_blocks",
    "swap_out_blocks",
    "swap_in_blocks",
    "block_bytes",
    "reshape_and_cache",
    "paged_attention_v1",
    "paged_attention_v2",
]


def _fail(msg: str) -> None:
    raise RuntimeError(msg)


def _stream_handle(device: torch.device, stream: Optional[torch.cuda.Stream]) -> int:
    return stream.cuda_stream if stream is not None else _lib.current_stream_handle(device)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _check_cuda(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            _fail(f"expected a GPU tensor, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            _fail(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def _check_cache(cache: torch.Tensor, name: str) -> None:
    if cache.dim() != 4:
        _fail(f"{name} must be [num_blocks, block_size, num_kv_heads, head_dim], got {tuple(cache.shape)}")
    if cache.stride(3) != 1 or cache.stride(2) != cache.shape[3]:
        _fail(f"{name}: the heads of a token must be contiguous (strides {cache.stride()})")


def _oob_ptr(oob_count: Optional[torch.Tensor]) -> Optional[int]:
    if oob_count is None:
        return None
    if oob_count.dtype != torch.int32 or oob_count.numel() < 1 or not oob_count.is_cuda:
        _fail("oob_count must be a GPU int32 tensor with at least one element")
    return oob_count.data_ptr()


# --------------------------------------------------------------------------
# (a5) KV append
# --------------------------------------------------------------------------
def reshape_and_cache_flash(key: torch.Tensor, value: torch.Tensor,
                            key_cache: torch.Tensor, value_cache: torch.Tensor,
                            slot_mapping: torch.Tensor, kv_cache_dtype: str = "auto",
                            k_scale: Optional[torch.Tensor] = None,
                            v_scale: Optional[torch.Tensor] = None, *,
                            oob_count: Optional[torch.Tensor] = None,
                            stream: Optional[torch.cuda.Stream] = None) -> None:
    """Write key[i]/value[i] into cache slot ``slot_mapping[i]`` (in place).

    Same contract as vLLM's ``reshape_and_cache_flash`` as the reference calls
    it (moe_engine.py:2059-2062): key/value ``[num_tokens, num_kv_heads,
    head_dim]``, caches ``[num_blocks, block_size, num_kv_heads, head_dim]``,
    int64 slot_mapping whose length is the token count (key may hold more
    rows), a negative slot is padding.  ``kv_cache_dtype`` must be "auto" (a
    plain copy, as in the engine, :454-457); the scales are then unused.
    """
    if kv_cache_dtype != "auto":
        _fail(f"kv_cache_dtype={kv_cache_dtype!r} is not supported (only 'auto')")
    dev = _check_cuda(key, value, key_cache, value_cache, slot_mapping)
    _check_cache(key_cache, "key_cache")
    _check_cache(value_cache, "value_cache")
    if key_cache.shape != value_cache.shape or key_cache.stride() != value_cache.stride():
        _fail("key_cache and value_cache must have the same shape and strides")
    if key.dtype != key_cache.dtype or value.dtype != value_cache.dtype:
        _fail(f"dtype mismatch: key {key.dtype} vs cache {key_cache.dtype}")
    if slot_mapping.dtype != torch.int64 or slot_mapping.dim() != 1:
        _fail("slot_mapping must be a 1-D int64 tensor")
    if not slot_mapping.is_contiguous():
        _fail("slot_mapping must be contiguous")
    nb, bs, h, d = key_cache.shape
    n = slot_mapping.numel()
    for name, t in (("key", key), ("value", value)):
        if t.dim() != 3 or t.shape[1] != h or t.shape[2] != d:
            _fail(f"{name} must be [num_tokens, {h}, {d}], got {tuple(t.shape)}")
        if t.shape[0] < n:
            _fail(f"{name} has {t.shape[0]} rows but slot_mapping has {n}")
        if t.stride(2) != 1 or t.stride(1) != d:
            _fail(f"{name}: heads of a token must be contiguous (strides {t.stride()})")
    _lib.call("kvc_reshape_and_cache_flash",
              key.data_ptr(), value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
              slot_mapping.data_ptr(), n, h, d, bs, nb, key_cache.element_size(),
              key.stride(0), value.stride(0), key_cache.stride(0), key_cache.stride(1),
              _oob_ptr(oob_count), _stream_handle(dev, stream))


# --------------------------------------------------------------------------
# Block-table gather
# --------------------------------------------------------------------------
def gather_kv(key_cache: torch.Tensor, value_cache: torch.Tensor,
              block_table: torch.Tensor, cu_seq_lens: torch.Tensor,
              max_seq_len: int, out_key: Optional[torch.Tensor] = None,
              out_value: Optional[torch.Tensor] = None,
              seq_starts: Optional[torch.Tensor] = None, *,
              oob_count: Optional[torch.Tensor] = None,
              stream: Optional[torch.cuda.Stream] = None):
    """Pack each sequence's KV into contiguous rows.

    Row ``cu_seq_lens[b] + i`` of the outputs receives logical token
    ``seq_starts[b] + i`` of sequence ``b`` (block-table row ``b``), i.e. the
    closed form ``cache[bt[b, :nb]].flatten(0, 1)[start:start+len]``.
    ``max_seq_len`` (host int) must bound every length.  Returns
    ``(out_key, out_value)``, each ``[total_tokens, num_kv_heads, head_dim]``.
    """
    dev = _check_cuda(key_cache, value_cache, block_table, cu_seq_lens, seq_starts)
    _check_cache(key_cache, "key_cache")
    _check_cache(value_cache, "value_cache")
    if key_cache.stride() != value_cache.stride() or key_cache.shape != value_cache.shape:
        _fail("key_cache and value_cache must have the same shape and strides")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.stride(1) != 1:
        _fail("block_table must be a 2-D int32 tensor with contiguous rows")
    if cu_seq_lens.dtype != torch.int32 or not cu_seq_lens.is_contiguous():
        _fail("cu_seq_lens must be a contiguous int32 tensor")
    batch = cu_seq_lens.numel() - 1
    if batch < 0 or batch > block_table.shape[0]:
        _fail("cu_seq_lens must have batch+1 entries with batch <= block_table rows")
    if seq_starts is not None and (seq_starts.dtype != torch.int32 or seq_starts.numel() < batch):
        _fail("seq_starts must be an int32 tensor with batch entries")
    nb, bs, h, d = key_cache.shape
    if out_key is None or out_value is None:
        total = int(cu_seq_lens[-1].item()) if batch > 0 else 0
        if out_key is None:
            out_key = torch.empty(total, h, d, dtype=key_cache.dtype, device=dev)
        if out_value is None:
            out_value = torch.empty(total, h, d, dtype=value_cache.dtype, device=dev)
    for name, t in (("out_key", out_key), ("out_value", out_value)):
        if t.dim() != 3 or t.shape[1:] != (h, d) or t.stride(2) != 1 or t.stride(1) != d:
            _fail(f"{name} must be [tokens, {h}, {d}] with contiguous rows")
        if t.dtype != key_cache.dtype:
            _fail(f"{name} dtype {t.dtype} != cache dtype {key_cache.dtype}")
    if out_key.stride(0) != out_value.stride(0):
        _fail("out_key and out_value must share the token stride")
    # The kernel writes no row at or past out_rows (and counts such rows in
    # oob_count), whatever the device cu_seq_lens says.
    out_rows = min(out_key.shape[0], out_value.shape[0])
    _lib.call("kvc_gather_kv",
              key_cache.data_ptr(), value_cache.data_ptr(), block_table.data_ptr(),
              block_table.stride(0), block_table.shape[1], cu_seq_lens.data_ptr(),
              _ptr(seq_starts), batch, int(max_seq_len), h, d, bs, nb,
              key_cache.element_size(), key_cache.stride(0), key_cache.stride(1),
              out_key.data_ptr(), out_value.data_ptr(), out_key.stride(0), out_rows,
              _oob_ptr(oob_count), _stream_handle(dev, stream))
    return out_key, out_value


# --------------------------------------------------------------------------
# (a8) merge of two attention states
# --------------------------------------------------------------------------
def merge_attention_states(out1: torch.Tensor, lse1: torch.Tensor,
                           out2: torch.Tensor, lse2: torch.Tensor,
                           out: Optional[torch.Tensor] = None,
                           lse: Optional[torch.Tensor] = None, *,
                           stream: Optional[torch.cuda.Stream] = None):
    """Device twin of ``merge_attention_states`` (src/dense/offload_kv_attn.py:24-39):
    ``lse = logaddexp(lse1, lse2)``, ``out = out1*e^(lse1-lse) + out2*e^(lse2-lse)``
    in fp32, bf16 ``[..., head_dim]`` outputs, natural-log fp32 lse ``[...]``."""
    dev = _check_cuda(out1, lse1, out2, lse2)
    for t in (out1, out2):
        if t.dtype != torch.bfloat16 or not t.is_contiguous():
            _fail("out1/out2 must be contiguous bf16")
    if out1.shape != out2.shape or lse1.shape != out1.shape[:-1] or lse2.shape != lse1.shape:
        _fail("shape mismatch between outs and lses")
    if lse1.dtype != torch.float32 or lse2.dtype != torch.float32:
        _fail("lse1/lse2 must be float32")
    lse1 = lse1.contiguous()
    lse2 = lse2.contiguous()
    if out is None:
        out = torch.empty_like(out1)
    if lse is None:
        lse = torch.empty_like(lse1)
    d = out1.shape[-1]
    n = out1.numel() // d
    _lib.call("kvc_merge_attention_states", out1.data_ptr(), lse1.data_ptr(),
              out2.data_ptr(), lse2.data_ptr(), n, d, out.data_ptr(), lse.data_ptr(),
              _stream_handle(dev, stream))
    return out, lse


# --------------------------------------------------------------------------
# (f1) metadata
# --------------------------------------------------------------------------
def compute_slot_mapping(block_table: torch.Tensor, seq_ids: torch.Tensor,
                         query_start_loc: torch.Tensor, num_computed: torch.Tensor,
                         num_tokens: int, slot_mapping: torch.Tensor,
                         positions: Optional[torch.Tensor] = None,
                         block_size: int = 16, *,
                         stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """Positions and slots of a step's tokens, padded with -1 to
    ``slot_mapping.numel()`` (the engine's graph size), as vLLM's
    prepare_pos_seq_lens + _compute_slot_mappings_kernel compute them for the
    reference (moe_engine.py:3514-3541)."""
    dev = _check_cuda(block_table, seq_ids, query_start_loc, num_computed, slot_mapping, positions)
    for name, t in (("block_table", block_table), ("seq_ids", seq_ids),
                    ("query_start_loc", query_start_loc), ("num_computed", num_computed)):
        if t.dtype != torch.int32:
            _fail(f"{name} must be int32")
    if block_table.stride(1) != 1:
        _fail("block_table rows must be contiguous")
    if not (seq_ids.is_contiguous() and query_start_loc.is_contiguous() and num_computed.is_contiguous()):
        _fail("metadata tensors must be contiguous")
    if slot_mapping.dtype != torch.int64 or not slot_mapping.is_contiguous():
        _fail("slot_mapping must be contiguous int64")
    if positions is not None and (positions.dtype != torch.int32 or positions.numel() < slot_mapping.numel()):
        _fail("positions must be int32 with at least slot_mapping.numel() entries")
    num_reqs = seq_ids.numel()
    if query_start_loc.numel() < num_reqs + 1:
        _fail("query_start_loc needs num_reqs + 1 entries")
    if num_tokens > slot_mapping.numel():
        _fail("num_tokens exceeds slot_mapping length")
    _lib.call("kvc_compute_slot_mapping", block_table.data_ptr(), block_table.stride(0),
              block_table.shape[0], block_table.shape[1], seq_ids.data_ptr(),
              query_start_loc.data_ptr(), num_computed.data_ptr(), num_reqs, int(num_tokens),
              slot_mapping.numel(), int(block_size), slot_mapping.data_ptr(), _ptr(positions),
              _stream_handle(dev, stream))
    return slot_mapping


def copy_page_indices(block_table: torch.Tensor, indptr: torch.Tensor,
                      indices: torch.Tensor, seq_ids: Optional[torch.Tensor] = None, *,
                      stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """``indices[indptr[r]:indptr[r+1]] = block_table[seq_ids[r], :n_r]``
    (the reference's row index_select + _copy_page_indices_kernel,
    moe_engine.py:1937-1946).  ``indices`` must be contiguous; entries past
    its end are not written."""
    dev = _check_cuda(block_table, indptr, indices, seq_ids)
    if block_table.dtype != torch.int32 or block_table.stride(1) != 1:
        _fail("block_table must be int32 with contiguous rows")
    if indptr.dtype != torch.int32 or indices.dtype != torch.int32:
        _fail("indptr and indices must be int32")
    if seq_ids is not None and seq_ids.dtype != torch.int32:
        _fail("seq_ids must be int32")
    if not indices.is_contiguous():
        _fail("indices must be contiguous")
    num_reqs = indptr.numel() - 1
    _lib.call("kvc_copy_page_indices", block_table.data_ptr(), block_table.stride(0),
              block_table.shape[0], _ptr(seq_ids), indptr.data_ptr(), num_reqs,
              block_table.shape[1], indices.data_ptr(), indices.numel(),
              _stream_handle(dev, stream))
    return indices


def stage_from_host(host: torch.Tensor, dev: torch.Tensor, head: int,
                    tail_begin: int = 0, tail_end: int = 0, *,
                    stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """``dev[i] = host[i]`` for i in ``[0, head)`` and ``[tail_begin,
    tail_end)``: the engine's pinned-buffer uploads of step metadata
    (moe_engine.py:3493-3494, 3506-3507) as one kernel on the compute stream,
    which reads the pinned int32 ``host`` when it runs (keep it unchanged
    until then: record an event after the call)."""
    dev_ = _check_cuda(dev)
    if host.is_cuda or not host.is_pinned():
        _fail("host must be a pinned CPU tensor")
    if host.dtype != torch.int32 or dev.dtype != torch.int32:
        _fail("host and dev must be int32")
    if not (host.is_contiguous() and dev.is_contiguous()):
        _fail("host and dev must be contiguous")
    n = min(host.numel(), dev.numel())
    if tail_end == 0:
        tail_begin = tail_end = (head + 3) // 4 * 4      # no tail range
        if not 0 <= head <= n:
            _fail(f"range [0, {head}) does not fit host[{host.numel()}] / dev[{dev.numel()}]")
    elif not (0 <= head <= tail_begin <= tail_end <= n):
        _fail(f"ranges [0, {head}) and [{tail_begin}, {tail_end}) do not fit "
              f"host[{host.numel()}] / dev[{dev.numel()}]")
    _lib.call("kvc_stage_from_host", host.data_ptr(), dev.data_ptr(), head, tail_begin,
              tail_end, _stream_handle(dev_, stream))
    return dev


def decode_step_setup(host: torch.Tensor, dev: torch.Tensor, layout,
                      block_table: torch.Tensor, seq_lens: torch.Tensor,
                      slot_mapping: torch.Tensor, indices: torch.Tensor, *,
                      stream_handle: Optional[int] = None) -> None:
    """A pure-decode step's whole device setup in one launch
    (``kvc_decode_step_setup``): upload of the pinned int32 image ``host``
    into ``dev``, the block-table writes it lists, ``seq_lens``, the new
    tokens' slots (-1 padded to ``slot_mapping.numel()``) and the page-index
    flatten into ``indices`` -- the engine's setup sequence
    (moe_engine.py:3493-3556, 1937-1946).  ``layout`` is a
    ``_lib.KvcDecodeStepLayout``; ``host`` must stay unchanged until the
    kernel ran (record an event after the call).  The caller (the cache)
    builds every tensor, so only what the kernel indexes by is checked."""
    # (the library checks that host is pinned memory)
    if host.is_cuda or host.dtype != torch.int32:
        _fail("host must be a pinned int32 CPU tensor")
    if not (dev.dtype == torch.int32 and block_table.dtype == torch.int32
            and seq_lens.dtype == torch.int32 and indices.dtype == torch.int32
            and slot_mapping.dtype == torch.int64):
        _fail("dev, block_table, seq_lens and indices must be int32, slot_mapping int64")
    if layout.tail_end > min(host.numel(), dev.numel()):
        _fail("the layout's tail range does not fit the images")
    if (block_table.stride(1) != 1 or block_table.stride(0) != block_table.shape[1]
            or not (seq_lens.is_contiguous() and slot_mapping.is_contiguous()
                    and indices.is_contiguous())):
        _fail("block_table rows, seq_lens, slot_mapping and indices must be contiguous")
    if seq_lens.numel() < layout.max_seqs or slot_mapping.numel() < layout.num_reqs:
        _fail("seq_lens or slot_mapping too short for the layout")
    sh = (stream_handle if stream_handle is not None
          else _lib.current_stream_handle(dev.device))
    _lib.call("kvc_decode_step_setup", host.data_ptr(), dev.data_ptr(), layout,
              block_table.data_ptr(), block_table.stride(0), block_table.shape[0],
              block_table.shape[1], seq_lens.data_ptr(), slot_mapping.data_ptr(),
              slot_mapping.numel(), indices.data_ptr(), indices.numel(), sh)


# --------------------------------------------------------------------------
# (a10) block eviction / restore
# --------------------------------------------------------------------------
def block_bytes(cache: torch.Tensor) -> int:
    """Bytes of one block of one cache tensor (block_size*heads*dim*elem)."""
    _, bs, h, d = cache.shape
    return bs * h * d * cache.element_size()


def _block_geometry(key_cache: torch.Tensor, value_cache: torch.Tensor):
    _check_cache(key_cache, "key_cache")
    if key_cache.shape != value_cache.shape or key_cache.stride() != value_cache.stride():
        _fail("key_cache and value_cache must have the same shape and strides")
    nb, bs, h, d = key_cache.shape
    if key_cache.stride(1) != h * d:
        _fail("a block must be contiguous (token stride == heads*dim) for block copies")
    return nb, key_cache.stride(0) * key_cache.element_size(), block_bytes(key_cache)


def _check_ids(block_ids: torch.Tensor) -> None:
    if block_ids.dtype != torch.int32 or block_ids.dim() != 1 or not block_ids.is_contiguous():
        _fail("block_ids must be a contiguous 1-D int32 tensor")


def gather_blocks(key_cache: torch.Tensor, value_cache: torch.Tensor,
                  block_ids: torch.Tensor, staging: torch.Tensor, *,
                  oob_count: Optional[torch.Tensor] = None,
                  stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """staging[i] = (K block, V block) of block_ids[i]; staging is a byte
    tensor of at least ``n * 2 * block_bytes``."""
    dev = _check_cuda(key_cache, value_cache, block_ids, staging)
    _check_ids(block_ids)
    nb, stride, bb = _block_geometry(key_cache, value_cache)
    n = block_ids.numel()
    if staging.numel() * staging.element_size() < n * 2 * bb:
        _fail(f"staging holds {staging.numel() * staging.element_size()} bytes, need {n * 2 * bb}")
    _lib.call("kvc_gather_blocks", key_cache.data_ptr(), value_cache.data_ptr(), stride, bb,
              nb, block_ids.data_ptr(), n, staging.data_ptr(), _oob_ptr(oob_count),
              _stream_handle(dev, stream))
    return staging


def scatter_blocks(staging: torch.Tensor, block_ids: torch.Tensor,
                   key_cache: torch.Tensor, value_cache: torch.Tensor, *,
                   oob_count: Optional[torch.Tensor] = None,
                   stream: Optional[torch.cuda.Stream] = None) -> None:
    """Inverse of gather_blocks: block_ids[i] <- staging[i]."""
    dev = _check_cuda(key_cache, value_cache, block_ids, staging)
    _check_ids(block_ids)
    nb, stride, bb = _block_geometry(key_cache, value_cache)
    n = block_ids.numel()
    if staging.numel() * staging.element_size() < n * 2 * bb:
        _fail(f"staging holds {staging.numel() * staging.element_size()} bytes, need {n * 2 * bb}")
    _lib.call("kvc_scatter_blocks", staging.data_ptr(), block_ids.data_ptr(), n,
              key_cache.data_ptr(), value_cache.data_ptr(), stride, bb, nb,
              _oob_ptr(oob_count), _stream_handle(dev, stream))


def swap_out_blocks(key_caches: Sequence[torch.Tensor], value_caches: Sequence[torch.Tensor],
                    block_ids: torch.Tensor, host: torch.Tensor, staging: torch.Tensor, *,
                    oob_count: Optional[torch.Tensor] = None,
                    stream: Optional[torch.cuda.Stream] = None) -> None:
    """Copy blocks ``block_ids`` of every layer to pinned host memory.

    ``host`` is a pinned uint8 tensor viewed as ``[layers, n, 2, block_bytes]``;
    ``staging`` a device byte buffer (chunking happens when it is smaller than
    one layer's blocks).  Everything is enqueued on ``stream`` (default: the
    current stream); record an event on it to know when the host copy is whole.
    """
    if len(key_caches) != len(value_caches):
        _fail("key_caches and value_caches differ in length")
    dev = _check_cuda(block_ids, staging, *key_caches, *value_caches)
    _check_ids(block_ids)
    if host.is_cuda or not host.is_pinned():
        _fail("host buffer must be pinned CPU memory")
    n = block_ids.numel()
    if n == 0:
        return
    per_layer = None
    for layer, (kc, vc) in enumerate(zip(key_caches, value_caches)):
        nb, stride, bb = _block_geometry(kc, vc)
        per_layer = n * 2 * bb
        if host.numel() * host.element_size() < (layer + 1) * per_layer:
            _fail("host buffer too small for all layers")
        _lib.call("kvc_swap_out", kc.data_ptr(), vc.data_ptr(), stride, bb, nb,
                  block_ids.data_ptr(), n, staging.data_ptr(),
                  staging.numel() * staging.element_size(),
                  host.data_ptr() + layer * per_layer, _oob_ptr(oob_count),
                  _stream_handle(dev, stream))


def swap_in_blocks(host: torch.Tensor, block_ids: torch.Tensor,
                   key_caches: Sequence[torch.Tensor], value_caches: Sequence[torch.Tensor],
                   staging: torch.Tensor, *, oob_count: Optional[torch.Tensor] = None,
                   stream: Optional[torch.cuda.Stream] = None) -> None:
    """Restore blocks saved by swap_out_blocks into ``block_ids`` (which may
    differ from the ids they were evicted from)."""
    if len(key_caches) != len(value_caches):
        _fail("key_caches and value_caches differ in length")
    dev = _check_cuda(block_ids, staging, *key_caches, *value_caches)
    _check_ids(block_ids)
    if host.is_cuda or not host.is_pinned():
        _fail("host buffer must be pinned CPU memory")
    n = block_ids.numel()
    if n == 0:
        return
    for layer, (kc, vc) in enumerate(zip(key_caches, value_caches)):
        nb, stride, bb = _block_geometry(kc, vc)
        per_layer = n * 2 * bb
        if host.numel() * host.element_size() < (layer + 1) * per_layer:
            _fail("host buffer too small for all layers")
        _lib.call("kvc_swap_in", host.data_ptr() + layer * per_layer, block_ids.data_ptr(), n,
                  kc.data_ptr(), vc.data_ptr(), stride, bb, nb, staging.data_ptr(),
                  staging.numel() * staging.element_size(), _oob_ptr(oob_count),
                  _stream_handle(dev, stream))


# --------------------------------------------------------------------------
# (f3) vLLM's x-packed layout: reshape_and_cache + paged_attention_v1/v2
# --------------------------------------------------------------------------
_XDTYPES = {torch.float16: 0, torch.bfloat16: 1}


def _check_xpacked(key_cache: torch.Tensor, value_cache: torch.Tensor):
    """[nb, H, D/x, bs, x] and [nb, H, D, bs] with packed inner dimensions
    and equal block / head strides; returns (nb, H, D, bs, x)."""
    if key_cache.dim() != 5 or value_cache.dim() != 4:
        _fail("x-packed caches must be key [nb, H, D/x, bs, x] and value [nb, H, D, bs]")
    nb, h, dx, bs, x = key_cache.shape
    d = dx * x
    if tuple(value_cache.shape) != (nb, h, d, bs):
        _fail(f"value_cache must be [{nb}, {h}, {d}, {bs}], got {tuple(value_cache.shape)}")
    if key_cache.dtype not in _XDTYPES or value_cache.dtype != key_cache.dtype:
        _fail("x-packed caches must be float16 or bfloat16, both the same")
    if x != 16 // key_cache.element_size():
        _fail(f"x must be 16 bytes / element = {16 // key_cache.element_size()}, got {x}")
    if (key_cache.stride()[2:] != (bs * x, x, 1) or value_cache.stride()[2:] != (bs, 1)
            or key_cache.stride()[:2] != value_cache.stride()[:2]):
        _fail("x-packed caches: inner dimensions packed, block/head strides equal for K and V")
    return nb, h, d, bs, x


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                      value_cache: torch.Tensor, slot_mapping: torch.Tensor,
                      kv_cache_dtype: str = "auto", k_scale: Optional[torch.Tensor] = None,
                      v_scale: Optional[torch.Tensor] = None, *,
                      oob_count: Optional[torch.Tensor] = None,
                      stream: Optional[torch.cuda.Stream] = None) -> None:
    """vLLM's ``reshape_and_cache`` into the x-packed layout, as the dense
    sandbox calls it (src/dense/include/paged_transformer.py:290-294): key /
    value ``[num_tokens, H, D]`` (token stride free, heads packed), key_cache
    ``[nb, H, D/x, 16, x]``, value_cache ``[nb, H, D, 16]``; a negative slot is
    padding.  Bit copies; ``kv_cache_dtype`` must be "auto"."""
    if kv_cache_dtype != "auto":
        _fail(f"kv_cache_dtype={kv_cache_dtype!r} is not supported (only 'auto')")
    dev = _check_cuda(key, value, key_cache, value_cache, slot_mapping)
    nb, h, d, bs, x = _check_xpacked(key_cache, value_cache)
    if slot_mapping.dtype != torch.int64 or slot_mapping.dim() != 1 or not slot_mapping.is_contiguous():
        _fail("slot_mapping must be a contiguous 1-D int64 tensor")
    n = slot_mapping.numel()
    for name, t in (("key", key), ("value", value)):
        if t.dim() != 3 or tuple(t.shape[1:]) != (h, d) or t.shape[0] < n:
            _fail(f"{name} must be [>= {n}, {h}, {d}], got {tuple(t.shape)}")
        if t.stride(2) != 1 or t.stride(1) != d or t.dtype != key_cache.dtype:
            _fail(f"{name}: heads must be packed and the dtype must match the cache")
    _lib.call("kvc_reshape_and_cache_xpacked", key.data_ptr(), value.data_ptr(),
              key_cache.data_ptr(), value_cache.data_ptr(), slot_mapping.data_ptr(), n, h, d,
              bs, x, nb, key.stride(0), value.stride(0), key_cache.stride(0),
              key_cache.stride(1), _oob_ptr(oob_count), _stream_handle(dev, stream))


def _paged_attention(v2: bool, out, exp_sums, max_logits, tmp_out, query, key_cache,
                     value_cache, num_kv_heads, scale, block_tables, seq_lens, block_size,
                     max_seq_len, alibi_slopes, kv_cache_dtype, k_scale, v_scale, extra, stream):
    if alibi_slopes is not None:
        _fail("alibi_slopes are not supported")
    if kv_cache_dtype != "auto":
        _fail(f"kv_cache_dtype={kv_cache_dtype!r} is not supported (only 'auto')")
    if any(int(v) != 0 for v in extra[:2]) or (len(extra) > 3 and int(extra[3]) != 0):
        _fail("block-sparse attention is not supported")
    for sc in (k_scale, v_scale):
        if sc is not None and float(sc) != 1.0:
            _fail("k/v scales other than 1.0 are not supported (no fp8 cache)")
    dev = _check_cuda(out, query, key_cache, value_cache, block_tables, seq_lens,
                      exp_sums, max_logits, tmp_out)
    nb, hkv, d, bs, x = _check_xpacked(key_cache, value_cache)
    if hkv != num_kv_heads:
        _fail(f"num_kv_heads={num_kv_heads} but the cache holds {hkv} heads")
    if block_size != bs:
        _fail(f"block_size={block_size} but the cache blocks hold {bs} tokens")
    if query.dim() != 3 or query.shape[2] != d or query.dtype != key_cache.dtype:
        _fail(f"query must be [num_seqs, num_heads, {d}] of the cache dtype")
    seqs, hq = query.shape[0], query.shape[1]
    if query.stride(2) != 1 or query.stride(1) != d:
        _fail("query: heads must be packed")
    if tuple(out.shape) != (seqs, hq, d) or not out.is_contiguous() or out.dtype != query.dtype:
        _fail(f"out must be a contiguous [{seqs}, {hq}, {d}] tensor of the query dtype")
    if block_tables.dtype != torch.int32 or block_tables.dim() != 2 or block_tables.stride(1) != 1:
        _fail("block_tables must be int32 [num_seqs, max_blocks] with packed rows")
    if block_tables.shape[0] < seqs or seq_lens.dtype != torch.int32 or seq_lens.numel() < seqs:
        _fail("block_tables / seq_lens need one row / entry per sequence")
    if not seq_lens.is_contiguous():
        _fail("seq_lens must be contiguous")
    dt = _XDTYPES[key_cache.dtype]
    common = (query.data_ptr(), query.stride(0), key_cache.data_ptr(), value_cache.data_ptr(),
              seqs, hq, num_kv_heads, d, float(scale), block_tables.data_ptr(),
              block_tables.stride(0), block_tables.shape[1], seq_lens.data_ptr(), bs,
              int(max_seq_len), nb, dt, key_cache.stride(0), key_cache.stride(1),
              _stream_handle(dev, stream))
    if not v2:
        _lib.call("kvc_paged_attention_v1", out.data_ptr(), *common)
        return
    parts = exp_sums.shape[-1] if exp_sums.dim() == 3 else 0
    for name, t, shp in (("exp_sums", exp_sums, (seqs, hq, parts)),
                         ("max_logits", max_logits, (seqs, hq, parts)),
                         ("tmp_out", tmp_out, (seqs, hq, parts, d))):
        if tuple(t.shape) != shp or not t.is_contiguous():
            _fail(f"{name} must be a contiguous {shp} tensor")
    if exp_sums.dtype != torch.float32 or max_logits.dtype != torch.float32 \
            or tmp_out.dtype != query.dtype:
        _fail("exp_sums / max_logits are float32, tmp_out has the query dtype")
    _lib.call("kvc_paged_attention_v2", out.data_ptr(), exp_sums.data_ptr(),
              max_logits.data_ptr(), tmp_out.data_ptr(), parts, *common)


def paged_attention_v1(out: torch.Tensor, query: torch.Tensor, key_cache: torch.Tensor,
                       value_cache: torch.Tensor, num_kv_heads: int, scale: float,
                       block_tables: torch.Tensor, seq_lens: torch.Tensor, block_size: int,
                       max_seq_len: int, alibi_slopes: Optional[torch.Tensor] = None,
                       kv_cache_dtype: str = "auto", k_scale=None, v_scale=None,
                       tp_rank: int = 0, blocksparse_local_blocks: int = 0,
                       blocksparse_vert_stride: int = 0, blocksparse_block_size: int = 64,
                       blocksparse_head_sliding_step: int = 0, *,
                       stream: Optional[torch.cuda.Stream] = None) -> None:
    """vLLM's ``paged_attention_v1`` over the x-packed layout
    (src/dense/scratch_examples/vllm_paged_attn.py:274-279): one pass per
    (sequence, KV head) over the whole context, written to ``out``."""
    _paged_attention(False, out, None, None, None, query, key_cache, value_cache, num_kv_heads,
                     scale, block_tables, seq_lens, block_size, max_seq_len, alibi_slopes,
                     kv_cache_dtype, k_scale, v_scale,
                     (blocksparse_local_blocks, blocksparse_vert_stride, blocksparse_block_size,
                      blocksparse_head_sliding_step), stream)


def paged_attention_v2(out: torch.Tensor, exp_sums: torch.Tensor, max_logits: torch.Tensor,
                       tmp_out: torch.Tensor, query: torch.Tensor, key_cache: torch.Tensor,
                       value_cache: torch.Tensor, num_kv_heads: int, scale: float,
                       block_tables: torch.Tensor, seq_lens: torch.Tensor, block_size: int,
                       max_seq_len: int, alibi_slopes: Optional[torch.Tensor] = None,
                       kv_cache_dtype: str = "auto", k_scale=None, v_scale=None,
                       tp_rank: int = 0, blocksparse_local_blocks: int = 0,
                       blocksparse_vert_stride: int = 0, blocksparse_block_size: int = 64,
                       blocksparse_head_sliding_step: int = 0, *,
                       stream: Optional[torch.cuda.Stream] = None) -> None:
    """vLLM's ``paged_attention_v2`` over the x-packed layout, as the dense
    sandbox calls it (src/dense/include/paged_transformer.py:325-332): the
    context is cut into 512-token partitions whose max logit, exp-sum and
    normalised output land in ``max_logits`` / ``exp_sums`` / ``tmp_out``
    ([num_seqs, num_heads, partitions(, D)], partitions >=
    ceil(max_seq_len / 512)), then combined into ``out``."""
    _paged_attention(True, out, exp_sums, max_logits, tmp_out, query, key_cache, value_cache,
                     num_kv_heads, scale, block_tables, seq_lens, block_size, max_seq_len,
                     alibi_slopes, kv_cache_dtype, k_scale, v_scale,
                     (blocksparse_local_blocks, blocksparse_vert_stride, blocksparse_block_size,
                      blocksparse_head_sliding_step), stream)
