"""Paged GQA decode attention with FlashInfer's wrapper interface.

``BatchDecodeWithPagedKVCacheWrapper`` keeps the constructor / ``plan`` /
``run`` signature the reference engine uses
(src/MoE/moe_engine.py:551-552 construct, :1352-1358 and :1949-1955 plan,
:2069-2070 and :3907-3909 run) and launches the HIP kernels of
csrc/decode.hip through libkvc.so.

``plan`` is host work (plus one small H2D copy), like FlashInfer's: it reads
the host indptr, cuts the batch's pages into segments of equal cost (the
balanced split-KV schedule of kvc_decode_plan) and stages the schedule, indptr, indices
and last_page_len on the device.  ``run`` launches the streaming kernel and,
when a request spans more than one segment, the merge kernel.  ``plan`` must be
called again whenever the sequence lengths change (the engine re-plans every
step after bumping ``_seq_lens_cpu``, moe_engine.py:3554-3556).
"""
from __future__ import annotations

import math
import weakref
from typing import Optional, Tuple, Union

import numpy as np
import torch

from . import _lib

__all__ = ["BatchDecodeWithPagedKVCacheWrapper"]

_DEFAULT_WORKSPACE = 128 * 1024 * 1024  # the engine's FlashInfer workspace (moe_engine.py:541-542)


def _fail(msg: str) -> None:
    raise RuntimeError(msg)


class BatchDecodeWithPagedKVCacheWrapper:
    """Decode attention over a paged KV cache ("NHD" layout).

    Parameters mirror FlashInfer's wrapper.  ``float_workspace_buffer`` is a
    device byte buffer that holds split-K partials (FlashInfer's engine call
    passes 128 MiB); ``plan`` raises if a batch needs more.
    """

    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD",
                 use_cuda_graph: bool = False, use_tensor_cores: bool = False,
                 paged_kv_indptr_buffer: Optional[torch.Tensor] = None,
                 paged_kv_indices_buffer: Optional[torch.Tensor] = None,
                 paged_kv_last_page_len_buffer: Optional[torch.Tensor] = None,
                 num_segments: Optional[int] = None):
        if kv_layout != "NHD":
            _fail(f"kv_layout={kv_layout!r} is not supported (only 'NHD')")
        if use_cuda_graph:
            # FlashInfer's graph mode re-plans into fixed buffers between
            # replays; here plan() stages a new schedule image per call (a
            # captured run() stays valid only until the next plan()).  The
            # engine constructs its wrapper with use_cuda_graph=False
            # (moe_engine.py:551-552).
            _fail("use_cuda_graph=True is not supported (capture run() within one plan instead)")
        if not float_workspace_buffer.is_cuda:
            _fail("float_workspace_buffer must be a GPU tensor")
        self._workspace = float_workspace_buffer
        self._device = float_workspace_buffer.device
        self._use_cuda_graph = use_cuda_graph
        self._indptr_buf = paged_kv_indptr_buffer
        self._indices_buf = paged_kv_indices_buffer
        self._lpl_buf = paged_kv_last_page_len_buffer
        self._segments_hint = int(num_segments or 0)
        self._dev_index = self._device.index if self._device.index is not None \
            else torch.cuda.current_device()
        self._num_cus = torch.cuda.get_device_properties(self._device).multi_processor_count
        self._sched: Optional[_lib.KvcDecodeSchedule] = None
        self._indices = None
        self._num_indices = 0
        self._sm_scale = None
        self._plan_args = None
        # (id(k), id(v)) -> (k ref, v ref, (ps, hkv, d), launch arguments)
        # for the cache tensors already checked (one pair per layer).
        self._kv_checked: dict = {}
        self._fused_ok = False
        self._cap_cache: dict = {}   # batch -> plan-image capacity
        ws = float_workspace_buffer
        self._ws_args = (ws.data_ptr(), ws.numel() * ws.element_size())
        self._meta_refs = None   # the tensors _meta_args was made from

    # ------------------------------------------------------------------ plan
    def plan(self, indptr: torch.Tensor, indices: torch.Tensor, last_page_len: torch.Tensor,
             num_qo_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
             pos_encoding_mode: str = "NONE", window_left: int = -1,
             logits_soft_cap: Optional[float] = None,
             q_data_type: Union[str, torch.dtype] = torch.bfloat16,
             kv_data_type: Optional[Union[str, torch.dtype]] = None,
             data_type: Optional[Union[str, torch.dtype]] = None,
             sm_scale: Optional[float] = None, rope_scale: Optional[float] = None,
             rope_theta: Optional[float] = None, non_blocking: bool = True) -> None:
        """Stage the batch metadata and choose the split-K schedule.

        indptr ``[B+1]`` int32 (page offsets), indices ``[indptr[B]]`` int32
        (physical page ids), last_page_len ``[B]`` int32 (1..page_size tokens
        in each request's final page).  Host or device tensors are accepted;
        the schedule is computed from a host copy of indptr.
        """
        if pos_encoding_mode != "NONE":
            _fail(f"pos_encoding_mode={pos_encoding_mode!r} not supported (engine uses 'NONE')")
        if window_left != -1 or logits_soft_cap not in (None, 0, 0.0):
            _fail("sliding windows and logits soft-cap are not supported")
        for dt in (q_data_type, kv_data_type, data_type):
            if dt is not None and dt not in (torch.bfloat16, "bfloat16", "bf16"):
                _fail(f"only bfloat16 q/kv are supported, got {dt}")
        if page_size != 16:
            _fail("page_size must be 16")
        if num_qo_heads % num_kv_heads != 0:
            _fail("num_qo_heads must be a multiple of num_kv_heads")
        for name, t in (("indptr", indptr), ("indices", indices), ("last_page_len", last_page_len)):
            if t.dtype != torch.int32:
                _fail(f"{name} must be int32")
        batch = indptr.numel() - 1
        if batch < 0:
            _fail("indptr must have at least one entry")
        if last_page_len.numel() < batch:
            _fail("last_page_len needs one entry per request")

        indptr_host = indptr[: batch + 1].to("cpu").contiguous() if indptr.is_cuda \
            else indptr[: batch + 1].contiguous()
        lpl_host = last_page_len[:batch].to("cpu").contiguous() if last_page_len.is_cuda \
            else last_page_len[:batch].contiguous()
        total = int(indptr_host[-1]) if batch > 0 else 0
        if indices.numel() < total:
            _fail(f"indices has {indices.numel()} entries, indptr[-1] = {total}")

        # Host-side schedule (kvc_decode_plan), written straight into the
        # pinned staging tensor of the one H2D copy of the batch metadata:
        #   [plan image | indptr | last_page_len].  A fresh pinned tensor from
        # torch's caching host allocator stays alive until its async copy has
        # run, so plan() never waits for the GPU.
        lib = _lib.load()
        sched = _lib.KvcDecodeSchedule()
        cap = lib.kvc_decode_plan_ints(batch, max(self._segments_hint, 8 * self._num_cus))
        for _ in range(2):
            cap4 = (cap + 3) // 4 * 4
            hs = torch.empty(cap4 + 2 * batch + 1, dtype=torch.int32, pin_memory=True)
            st = lib.kvc_decode_plan(indptr_host.data_ptr(), lpl_host.data_ptr(), batch,
                                     num_qo_heads, num_kv_heads,
                                     head_dim, page_size, self._segments_hint, self._num_cus,
                                     sched, hs.data_ptr(), cap4)
            if st == _lib.KVC_ERR_WORKSPACE and sched.plan_ints > cap4:
                cap = sched.plan_ints
                continue
            _lib.check("kvc_decode_plan", st)
            break
        ws = self._workspace.numel() * self._workspace.element_size()
        if sched.workspace_bytes > ws:
            _fail(f"decode workspace too small: need {sched.workspace_bytes} bytes, have {ws}")

        dev = self._device
        hs[cap4: cap4 + batch + 1].copy_(indptr_host)
        hs[cap4 + batch + 1:].copy_(lpl_host)
        dm = hs.to(dev, non_blocking=True)
        plan_dev = dm[:cap4]
        if self._indptr_buf is not None:
            self._indptr_buf[: batch + 1].copy_(dm[cap4: cap4 + batch + 1])
            indptr_dev = self._indptr_buf
        else:
            indptr_dev = dm[cap4: cap4 + batch + 1]
        if self._lpl_buf is not None:
            self._lpl_buf[:batch].copy_(dm[cap4 + batch + 1:])
            lpl_dev = self._lpl_buf
        else:
            lpl_dev = dm[cap4 + batch + 1:]
        if indices.is_cuda:
            if indices.device != dev:
                _fail("indices on a different device than the workspace")
            if self._indices_buf is not None:
                self._indices_buf[:total].copy_(indices[:total])
                indices_dev = self._indices_buf
            else:
                indices_dev = indices
        else:
            host_idx = indices[:total]
            if not host_idx.is_pinned():
                host_idx = host_idx.pin_memory()
            indices_dev = host_idx.to(dev, non_blocking=True)
        if not indices_dev.is_contiguous():
            indices_dev = indices_dev.contiguous()

        self._adopt(sched, plan_dev, indptr_dev, lpl_dev, indices_dev,
                    float(sm_scale) if sm_scale is not None else 1.0 / math.sqrt(head_dim),
                    (batch, num_qo_heads, num_kv_heads, head_dim, page_size))

    begin_forward = plan

    def _adopt(self, sched, plan_dev, indptr_dev, lpl_dev, indices_dev, sm_scale, plan_args):
        """Make a staged schedule current and precompute the parts of the
        launch arguments that stay fixed until the next plan."""
        self._sched = sched
        self._plan_dev = plan_dev
        self._indptr = indptr_dev
        self._lpl = lpl_dev
        self._indices = indices_dev
        self._num_indices = indices_dev.numel()
        self._sm_scale = sm_scale
        self._plan_args = plan_args
        self._pre_args = (sched, plan_dev.data_ptr())
        r = self._meta_refs
        if r is None or r[0] is not indptr_dev or r[1] is not indices_dev or r[2] is not lpl_dev:
            self._meta_refs = (indptr_dev, indices_dev, lpl_dev)
            self._meta_args = (indptr_dev.data_ptr(), indices_dev.data_ptr(),
                               self._num_indices, lpl_dev.data_ptr())
        self._fused_ok = (sched.head_dim == 128 and
                          (sched.small_batch == 1 or
                           (sched.heads_per_group == 8 and sched.append_pieces <= 4)))

    # ------------------------------------------------- in-package fast path
    def _plan_capacity(self, batch: int) -> int:
        """int32 entries to reserve for the plan image (16-byte multiple)."""
        cap = self._cap_cache.get(batch)
        if cap is None:
            cap = _lib.load().kvc_decode_plan_ints(batch,
                                                   max(self._segments_hint, 8 * self._num_cus))
            cap = (cap + 3) // 4 * 4
            if len(self._cap_cache) > 4096:
                self._cap_cache.clear()
            self._cap_cache[batch] = cap
        return cap

    def _schedule_into(self, indptr_host: np.ndarray, lpl_host: np.ndarray, batch: int,
                       num_qo_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
                       image) -> _lib.KvcDecodeSchedule:
        """kvc_decode_plan into the int32 ``image`` (a pinned tensor or a
        numpy view of one).  If the image is too small, the returned
        schedule's ``plan_ints`` exceeds its size and nothing is staged:
        retry with a larger one."""
        if isinstance(image, np.ndarray):
            ptr, size = image.ctypes.data, image.size
        else:
            ptr, size = image.data_ptr(), image.numel()
        sched = _lib.KvcDecodeSchedule()
        st = _lib.load().kvc_decode_plan(indptr_host.ctypes.data, lpl_host.ctypes.data, batch,
                                         num_qo_heads, num_kv_heads, head_dim, page_size,
                                         self._segments_hint, self._num_cus, sched, ptr, size)
        if st == _lib.KVC_ERR_WORKSPACE and sched.plan_ints > size:
            return sched
        _lib.check("kvc_decode_plan", st)
        ws = self._workspace.numel() * self._workspace.element_size()
        if sched.workspace_bytes > ws:
            _fail(f"decode workspace too small: need {sched.workspace_bytes} bytes, have {ws}")
        return sched

    def _install(self, sched: _lib.KvcDecodeSchedule, plan_dev: torch.Tensor,
                 indptr_dev: torch.Tensor, lpl_dev: torch.Tensor, indices_dev: torch.Tensor,
                 num_qo_heads: int, num_kv_heads: int, head_dim: int, page_size: int) -> None:
        """Adopt a schedule whose image and metadata are already on the device
        (staged by the caller in stream order before the next ``run``)."""
        self._adopt(sched, plan_dev, indptr_dev, lpl_dev, indices_dev, 1.0 / math.sqrt(head_dim),
                    (sched.batch, num_qo_heads, num_kv_heads, head_dim, page_size))

    @property
    def schedule(self) -> _lib.KvcDecodeSchedule:
        return self._sched

    # ------------------------------------------------------------------- run
    def run(self, q: torch.Tensor,
            paged_kv_cache: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
            *args, out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
            return_lse: bool = False, q_scale: Optional[float] = None,
            k_scale: Optional[float] = None, v_scale: Optional[float] = None,
            stream: Optional[torch.cuda.Stream] = None, **kwargs):
        """Attention of ``q [B, num_qo_heads, head_dim]`` over the planned pages.

        ``paged_kv_cache`` is ``(k_cache, v_cache)`` each
        ``[num_pages, page_size, num_kv_heads, head_dim]``, or one tensor
        ``[num_pages, 2, page_size, num_kv_heads, head_dim]``.  Returns ``out``
        (bf16 ``[B, num_qo_heads, head_dim]``) or ``(out, lse)``; lse is the
        natural-log log-sum-exp of the scaled logits.
        """
        if q_scale not in (None, 1.0) or k_scale not in (None, 1.0) or v_scale not in (None, 1.0):
            _fail("q/k/v scales are not supported (bf16 cache)")
        sh = (stream.cuda_stream if stream is not None
              else _lib.current_stream_handle(self._device))
        return self._launch(q, paged_kv_cache, out, lse, return_lse, sh, None, None)

    forward = run

    @property
    def fused_append_supported(self) -> bool:
        """Whether ``run_with_append`` can serve the planned batch (head_dim
        128 and either a small-batch schedule or 8 KV heads per workgroup
        with few request ends per segment)."""
        return self._sched is not None and self._fused_ok

    def run_with_append(self, q: torch.Tensor,
                        paged_kv_cache: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
                        new_key: torch.Tensor, new_value: torch.Tensor, *,
                        out: Optional[torch.Tensor] = None, lse: Optional[torch.Tensor] = None,
                        return_lse: bool = False, stream: Optional[torch.cuda.Stream] = None):
        """``run`` that first writes ``new_key[b]`` / ``new_value[b]``
        (``[B, num_kv_heads, head_dim]`` bf16) into the cache as request b's
        last token -- the slot a pure-decode step's slot mapping gives it --
        in the same launch (``kvc_batch_decode_append_run``).  Cache and
        output equal ``reshape_and_cache_flash`` followed by ``run`` bit for
        bit.  Raises unless ``fused_append_supported``."""
        sh = (stream.cuda_stream if stream is not None
              else _lib.current_stream_handle(self._device))
        return self._launch(q, paged_kv_cache, out, lse, return_lse, sh, new_key, new_value)

    def _launch(self, q, paged_kv_cache, out, lse, return_lse, sh, new_key, new_value,
                kv=None):
        """Check the call's tensors against the plan and launch the decode
        (with the fused append when ``new_key`` is given) on stream ``sh``.
        The plan's and the cache's arguments were checked and converted once
        (``_adopt``, ``_kv_args``); per call only q, out, lse and the new rows
        are checked.  ``kv``: the cache's launch arguments, already checked
        (``PagedKVCache`` passes those of its own layers)."""
        if self._sched is None:
            _fail("run() called before plan()")
        if kv is None:
            kv = self._kv_args(paged_kv_cache)
        batch, hq, hkv, d, ps = self._plan_args
        dev = self._dev_index
        qs, qt = q.shape, q.stride()
        if (len(qs) != 3 or qs[0] < batch or qs[1] != hq or qs[2] != d
                or q.dtype is not torch.bfloat16 or qt[2] != 1 or qt[1] != d):
            _fail(f"q must be bfloat16 [{batch}, {hq}, {d}] with contiguous heads, "
                  f"got {q.dtype} {tuple(qs)} strides {qt}")
        if q.get_device() != dev:
            _fail("q on a different device than the workspace")
        if out is None:
            out = torch.empty(batch, hq, d, dtype=torch.bfloat16, device=self._device)
        else:
            os_, ot = out.shape, out.stride()
            if (len(os_) != 3 or os_[0] < batch or os_[1] != hq or os_[2] != d
                    or out.dtype is not torch.bfloat16 or ot[2] != 1 or ot[1] != d
                    or out.get_device() != dev):
                _fail("out must be bfloat16 [B, num_qo_heads, head_dim] with contiguous heads "
                      "on the workspace's device")
        if return_lse and lse is None:
            lse = torch.empty(batch, hq, dtype=torch.float32, device=self._device)
        if lse is not None and (lse.dtype is not torch.float32 or not lse.is_contiguous()
                                or lse.numel() < batch * hq or lse.get_device() != dev):
            _fail("lse must be contiguous float32 [B, num_qo_heads] on the workspace's device")
        lse_p = lse.data_ptr() if lse is not None else None
        if new_key is None:
            _lib.call("kvc_batch_decode_run", *self._pre_args, q.data_ptr(), qt[0], *kv,
                      *self._meta_args, self._sm_scale, *self._ws_args, out.data_ptr(),
                      out.stride(0), lse_p, sh)
            return (out, lse) if return_lse else out
        if not self._fused_ok:
            _fail("the fused append needs head_dim 128, num_kv_heads a multiple of 8, "
                  "group <= 4 and at most 4 request ends in a segment's leading pieces")
        for name, t in (("new_key", new_key), ("new_value", new_value)):
            ts, tt = t.shape, t.stride()
            if (t.dtype is not torch.bfloat16 or len(ts) != 3 or ts[0] < batch
                    or ts[1] != hkv or ts[2] != d or tt[2] != 1 or tt[1] != d):
                _fail(f"{name} must be bfloat16 [B, {hkv}, {d}] with contiguous heads")
            if t.get_device() != dev:
                _fail(f"{name} on a different device than the workspace")
        _lib.call("kvc_batch_decode_append_run", *self._pre_args, q.data_ptr(), qt[0], *kv,
                  *self._meta_args, new_key.data_ptr(), new_key.stride(0), new_value.data_ptr(),
                  new_value.stride(0), self._sm_scale, *self._ws_args, out.data_ptr(),
                  out.stride(0), lse_p, sh)
        return (out, lse) if return_lse else out

    def _kv_args(self, paged_kv_cache):
        """(k ptr, v ptr, block stride, token stride, blocks) of the cache
        pair, checked against the plan's (page_size, heads, dim).  The
        per-layer cache views are the same tensor objects call after call:
        once checked they are recognised by identity, storage address and
        block count."""
        batch, hq, hkv, d, ps = self._plan_args
        if isinstance(paged_kv_cache, (tuple, list)):
            k_cache, v_cache = paged_kv_cache
        else:
            if paged_kv_cache.dim() != 5 or paged_kv_cache.shape[1] != 2:
                _fail("a single paged_kv_cache tensor must be [pages, 2, page_size, heads, dim]")
            k_cache, v_cache = paged_kv_cache[:, 0], paged_kv_cache[:, 1]
        seen = self._kv_checked.get((id(k_cache), id(v_cache)))
        if (seen is not None and seen[0]() is k_cache and seen[1]() is v_cache
                and seen[2] == (ps, hkv, d) and seen[3][0] == k_cache.data_ptr()
                and seen[3][4] == k_cache.shape[0] and seen[3][1] == v_cache.data_ptr()
                and v_cache.shape[0] == seen[3][4]):
            return seen[3]
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
        if len(self._kv_checked) >= 1024:
            self._kv_checked.clear()
        kv = (k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
              k_cache.shape[0])
        self._kv_checked[(id(k_cache), id(v_cache))] = (
            weakref.ref(k_cache), weakref.ref(v_cache), (ps, hkv, d), kv)
        return kv

    def end_forward(self) -> None:
        """No-op kept for interface parity."""
