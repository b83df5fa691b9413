"""Paged-KV prefill attention with FlashInfer's wrapper interface.

``BatchPrefillWithPagedKVCacheWrapper`` keeps the constructor / ``plan`` /
``run`` signature the reference engine uses for continuation prefills
(src/MoE/moe_engine.py:1733-1751 and :3710-3727 plan, :3939-3941 run) and
launches the MFMA kernel of csrc/prefill.hip through libkvc.so.

A continuation chunk's K/V are appended to the cache first (``slot_mapping``
append), so each request's keys are ``kv_len`` cached tokens of which the last
``q_len`` are the chunk's own.  With ``causal=True`` query i sees keys
``j <= i + kv_len - q_len`` (the mask is aligned to the end of the cache, as
FlashInfer's).

``plan`` is host work plus one small H2D copy: it reads the host index
pointers, cuts every request's queries into 256-row tiles (tile tokens x the
GQA group) ordered longest-first, and stages the work list.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple, Union

import numpy as np
import torch

from . import _lib

__all__ = ["BatchPrefillWithPagedKVCacheWrapper"]

# Query rows (tokens x the GQA group) per work item of the prefill kernel,
# and its most workgroups (one per CU; each runs a list of work items).
_TILE_ROWS = 256
_MAX_WORKGROUPS = 256


def _fail(msg: str) -> None:
    raise RuntimeError(msg)


def _host_int32(t: torch.Tensor, n: int, name: str) -> np.ndarray:
    if t.dtype != torch.int32:
        _fail(f"{name} must be int32")
    if t.numel() < n:
        _fail(f"{name} needs {n} entries, has {t.numel()}")
    return t[:n].detach().to("cpu").contiguous().numpy()


class BatchPrefillWithPagedKVCacheWrapper:
    """Prefill attention of multi-token queries over a paged KV cache ("NHD").

    ``float_workspace_buffer`` only fixes the device (the kernel keeps no
    split-K partials); it is accepted for interface parity.
    """

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, **kwargs):
        if kv_layout != "NHD":
            _fail(f"kv_layout={kv_layout!r} is not supported (only 'NHD')")
        if use_cuda_graph:
            _fail("use_cuda_graph=True is not supported (capture run() within one plan instead)")
        if not float_workspace_buffer.is_cuda:
            _fail("float_workspace_buffer must be a GPU tensor")
        self._device = float_workspace_buffer.device
        self._sched: Optional[_lib.KvcPrefillSchedule] = None
        self._plan_dev = None
        self._indices = None
        self._plan_args = None
        self._sm_scale = None

    def plan(self, qo_indptr: torch.Tensor, paged_kv_indptr: torch.Tensor,
             paged_kv_indices: torch.Tensor, paged_kv_last_page_len: torch.Tensor,
             num_qo_heads: int, num_kv_heads: int, head_dim_qk: int, page_size: int,
             head_dim_vo: Optional[int] = None, custom_mask: Optional[torch.Tensor] = None,
             packed_custom_mask: Optional[torch.Tensor] = None, causal: bool = False,
             pos_encoding_mode: str = "NONE", use_fp16_qk_reduction: bool = False,
             sm_scale: Optional[float] = None, window_left: int = -1,
             logits_soft_cap: Optional[float] = None, rope_scale: Optional[float] = None,
             rope_theta: Optional[float] = None,
             q_data_type: Union[str, torch.dtype] = torch.bfloat16,
             kv_data_type: Optional[Union[str, torch.dtype]] = None,
             non_blocking: bool = True, **kwargs) -> None:
        """Stage the work list for ``run``.  Index tensors may live on the host
        or the device (the schedule is computed from host copies, as
        FlashInfer's plan does)."""
        if head_dim_vo not in (None, head_dim_qk):
            _fail("head_dim_vo must equal head_dim_qk")
        if custom_mask is not None or packed_custom_mask is not None:
            _fail("custom masks are not supported")
        if pos_encoding_mode != "NONE" or window_left != -1 or logits_soft_cap not in (None, 0, 0.0):
            _fail("only pos_encoding_mode='NONE' without window or soft-cap is supported")
        for dt in (q_data_type, kv_data_type):
            if dt is not None and dt not in (torch.bfloat16, "bfloat16", "bf16"):
                _fail(f"only bfloat16 q/kv are supported, got {dt}")
        batch = qo_indptr.numel() - 1
        if batch < 0:
            _fail("qo_indptr must have at least one entry")
        if paged_kv_indptr.numel() != batch + 1:
            _fail("qo_indptr and paged_kv_indptr must have the same length")
        qo = _host_int32(qo_indptr, batch + 1, "qo_indptr")
        kv = _host_int32(paged_kv_indptr, batch + 1, "paged_kv_indptr")
        lpl = _host_int32(paged_kv_last_page_len, batch, "paged_kv_last_page_len")
        if paged_kv_indices.dtype != torch.int32:
            _fail("paged_kv_indices must be int32")
        total_pages = int(kv[-1]) if batch > 0 else 0
        if paged_kv_indices.numel() < total_pages:
            _fail(f"paged_kv_indices has {paged_kv_indices.numel()} entries, "
                  f"paged_kv_indptr[-1] = {total_pages}")
        if num_kv_heads <= 0 or num_qo_heads % num_kv_heads:
            _fail("num_qo_heads must be a multiple of num_kv_heads")
        group = num_qo_heads // num_kv_heads
        q_lens = np.diff(qo.astype(np.int64)) if batch > 0 else np.zeros(0, np.int64)
        cap = self._plan_capacity(q_lens, group, num_kv_heads)

        sched = _lib.KvcPrefillSchedule()
        hs = torch.empty(cap, dtype=torch.int32, pin_memory=True)
        _lib.call("kvc_prefill_plan", qo.ctypes.data, kv.ctypes.data, lpl.ctypes.data, batch,
                  num_qo_heads, num_kv_heads, head_dim_qk, page_size, 1 if causal else 0,
                  sched, hs.data_ptr(), cap)
        self._plan_dev = hs[: max(sched.plan_ints, 8)].to(self._device, non_blocking=True)
        idx = paged_kv_indices[:total_pages]
        if idx.is_cuda:
            if idx.device != self._device:
                _fail("paged_kv_indices on a different device than the workspace")
            idx = idx.contiguous()
        else:
            idx = idx.contiguous().pin_memory().to(self._device, non_blocking=True)
        self._indices = idx
        self._sched = sched
        self._plan_args = (int(qo[-1]) if batch > 0 else 0, num_qo_heads, num_kv_heads,
                           head_dim_qk, page_size)
        self._sm_scale = float(sm_scale) if sm_scale is not None else 1.0 / math.sqrt(head_dim_qk)

    begin_forward = plan

    # ------------------------------------------------- in-package fast path
    @staticmethod
    def _plan_capacity(q_lens: np.ndarray, group: int, num_kv_heads: int) -> int:
        """int32 entries to reserve for the plan image (16-byte multiple): the
        workgroups' (first unit, units) table, padded to 4 entries, and one
        8-entry record per (query tile, KV head)."""
        tile = _TILE_ROWS // group if group in (1, 2, 4, 8) else 1
        ql = np.maximum(np.asarray(q_lens, np.int64), 0)
        units = int(np.sum((ql + tile - 1) // tile)) * max(int(num_kv_heads), 1)
        table = (2 * min(_MAX_WORKGROUPS, units) + 3) // 4 * 4
        return table + 8 * units + 8

    def _schedule_into(self, qo: np.ndarray, kv: np.ndarray, lpl: np.ndarray, batch: int,
                       num_qo_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
                       causal: bool, image: torch.Tensor) -> _lib.KvcPrefillSchedule:
        """kvc_prefill_plan into the pinned int32 ``image`` (sized by
        ``_plan_capacity``)."""
        sched = _lib.KvcPrefillSchedule()
        _lib.call("kvc_prefill_plan", qo.ctypes.data, kv.ctypes.data, lpl.ctypes.data, batch,
                  num_qo_heads, num_kv_heads, head_dim, page_size, 1 if causal else 0,
                  sched, image.data_ptr(), image.numel())
        return sched

    def _install(self, sched: _lib.KvcPrefillSchedule, plan_dev: torch.Tensor,
                 indices_dev: torch.Tensor, total_q: int, num_qo_heads: int, num_kv_heads: int,
                 head_dim: int, page_size: int) -> None:
        """Adopt a schedule whose image and page indices are already on the
        device (staged by the caller in stream order before the next run)."""
        self._sched = sched
        self._plan_dev = plan_dev
        self._indices = indices_dev
        self._plan_args = (total_q, num_qo_heads, num_kv_heads, head_dim, page_size)
        self._sm_scale = 1.0 / math.sqrt(head_dim)

    @property
    def schedule(self) -> _lib.KvcPrefillSchedule:
        return self._sched

    def run(self, q: torch.Tensor,
            paged_kv_cache: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
            *args, out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
            return_lse: bool = False, k_scale: Optional[float] = None,
            v_scale: Optional[float] = None,
            stream: Optional[torch.cuda.Stream] = None, **kwargs):
        """Attention of ``q [total_q, num_qo_heads, head_dim]`` (the planned
        requests' query rows in ``qo_indptr`` order).  Returns ``out`` (bf16,
        same shape) or ``(out, lse)``."""
        if self._sched is None:
            _fail("run() called before plan()")
        if any(s not in (None, 1.0) for s in (k_scale, v_scale)):
            _fail("k/v scales are not supported (bf16 cache)")
        total_q, hq, hkv, d, ps = self._plan_args
        if isinstance(paged_kv_cache, (tuple, list)):
            k_cache, v_cache = paged_kv_cache
        else:
            if paged_kv_cache.dim() != 5 or paged_kv_cache.shape[1] != 2:
                _fail("a single paged_kv_cache tensor must be [pages, 2, page_size, heads, dim]")
            k_cache, v_cache = paged_kv_cache[:, 0], paged_kv_cache[:, 1]
        for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
            if c.dim() != 4 or tuple(c.shape[1:]) != (ps, hkv, d):
                _fail(f"{name} must be [pages, {ps}, {hkv}, {d}], got {tuple(c.shape)}")
            if c.dtype != torch.bfloat16:
                _fail(f"{name} must be bfloat16")
            if c.stride(3) != 1 or c.stride(2) != d:
                _fail(f"{name}: heads of a token must be contiguous")
            if c.device != self._device:
                _fail(f"{name} on {c.device}, workspace on {self._device}")
        if k_cache.stride() != v_cache.stride() or k_cache.shape[0] != v_cache.shape[0]:
            _fail("k_cache and v_cache must share shape and strides")
        if q.dim() != 3 or q.shape[0] < total_q or tuple(q.shape[1:]) != (hq, d):
            _fail(f"q must be [{total_q}, {hq}, {d}], got {tuple(q.shape)}")
        if q.dtype != torch.bfloat16 or q.stride(2) != 1 or q.stride(1) != d:
            _fail("q must be bfloat16 with contiguous heads")
        if q.device != self._device:
            _fail("q on a different device than the workspace")
        if out is None:
            out = torch.empty(total_q, hq, d, dtype=torch.bfloat16, device=self._device)
        elif (out.dtype != torch.bfloat16 or out.dim() != 3 or out.shape[0] < total_q
              or tuple(out.shape[1:]) != (hq, d) or out.stride(2) != 1 or out.stride(1) != d):
            _fail("out must be bfloat16 [total_q, num_qo_heads, head_dim] with contiguous heads")
        if return_lse and lse is None:
            lse = torch.empty(total_q, hq, dtype=torch.float32, device=self._device)
        if lse is not None and (lse.dtype != torch.float32 or not lse.is_contiguous()
                                or lse.numel() < total_q * hq):
            _fail("lse must be contiguous float32 [total_q, num_qo_heads]")
        sh = (stream.cuda_stream if stream is not None
              else _lib.current_stream_handle(self._device))
        _lib.call("kvc_batch_prefill_run", self._sched, self._plan_dev.data_ptr(),
                  q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
                  k_cache.stride(0), k_cache.stride(1), k_cache.shape[0],
                  self._indices.data_ptr(), self._indices.numel(), self._sm_scale,
                  out.data_ptr(), out.stride(0),
                  lse.data_ptr() if lse is not None else None, sh)
        return (out, lse) if return_lse else out

    forward = run

    def end_forward(self) -> None:
        """No-op kept for interface parity."""
