"""ctypes binding of libkvc.so, the C ABI declared in include/kvc.h.

The library is built in-tree (``gpu_offloading_amd/lib/libkvc.so``) by
``gpu_offloading_amd.build.build_library``.  There is no fallback: if the
library is missing every op raises ``RuntimeError``.

``torch`` is imported before the library is opened so that libkvc.so binds to
the HIP runtime torch already loaded (both carry the SONAME
``libamdhip64.so.7``); streams and device pointers handed over from torch are
then valid inside the library.
"""
from __future__ import annotations

import ctypes
import os
import threading
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_void_p

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")
LIB_PATH = os.path.join(LIB_DIR, "libkvc.so")

KVC_OK = 0
KVC_ERR_WORKSPACE = 4
STATUS_NAMES = {
    0: "KVC_OK",
    1: "KVC_ERR_INVALID_ARG",
    2: "KVC_ERR_UNSUPPORTED",
    3: "KVC_ERR_ALIGNMENT",
    4: "KVC_ERR_WORKSPACE",
    5: "KVC_ERR_HIP",
}


class KvcDecodeSchedule(ctypes.Structure):
    """Mirror of ``kvc_decode_schedule`` (include/kvc.h)."""

    _fields_ = [
        ("batch", c_int32),
        ("num_qo_heads", c_int32),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("page_size", c_int32),
        ("num_segments", c_int32),
        ("num_head_groups", c_int32),
        ("num_pieces", c_int32),
        ("pieces_offset", c_int32),
        ("nparts_offset", c_int32),
        ("max_partitions", c_int32),
        ("total_pages", c_int32),
        ("num_empty", c_int32),
        ("heads_per_group", c_int32),
        ("plan_ints", c_int64),
        ("workspace_bytes", c_int64),
        ("append_pieces", c_int32),
        ("small_batch", c_int32),
    ]


class KvcPrefillSchedule(ctypes.Structure):
    """Mirror of ``kvc_prefill_schedule`` (include/kvc.h)."""

    _fields_ = [
        ("batch", c_int32),
        ("num_qo_heads", c_int32),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("page_size", c_int32),
        ("causal", c_int32),
        ("tile_tokens", c_int32),
        ("num_items", c_int32),
        ("total_q", c_int32),
        ("max_key_tiles", c_int32),
        ("plan_ints", c_int64),
    ]


class KvcDecodeStepLayout(ctypes.Structure):
    """Mirror of ``kvc_decode_step_layout`` (include/kvc.h)."""

    _fields_ = [
        ("plan_ints", c_int64),
        ("tail_begin", c_int64),
        ("tail_end", c_int64),
        ("ids", c_int64),
        ("positions", c_int64),
        ("indptr", c_int64),
        ("lens_after", c_int64),
        ("bt_pos", c_int64),
        ("bt_val", c_int64),
        ("num_reqs", c_int32),
        ("num_bt_writes", c_int32),
        ("max_seqs", c_int32),
        ("block_size", c_int32),
    ]


_P = c_void_p
_I32P = c_void_p  # device int32 pointers are passed as raw addresses
# name -> (restype, argtypes).  Every entry point of include/kvc.h is listed;
# tests check this table against the header and the library's exports.
SIGNATURES = {
    "kvc_version": (c_int, []),
    "kvc_status_string": (c_char_p, [c_int]),
    "kvc_last_error": (c_char_p, []),
    "kvc_reshape_and_cache_flash": (c_int, [
        _P, _P, _P, _P, _P,
        c_int64, c_int32, c_int32, c_int32, c_int64, c_int32,
        c_int64, c_int64, c_int64, c_int64,
        _I32P, _P]),
    "kvc_gather_kv": (c_int, [
        _P, _P, _I32P, c_int64, c_int32, _I32P, _I32P,
        c_int32, c_int32, c_int32, c_int32, c_int32, c_int64, c_int32,
        c_int64, c_int64, _P, _P, c_int64, c_int64, _I32P, _P]),
    "kvc_decode_plan_ints": (c_int64, [c_int32, c_int32]),
    "kvc_decode_plan": (c_int, [
        c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
        POINTER(KvcDecodeSchedule), c_void_p, c_int64]),
    "kvc_decode_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32, c_int32]),
    "kvc_batch_decode_run": (c_int, [
        POINTER(KvcDecodeSchedule), _I32P, _P, c_int64, _P, _P, c_int64, c_int64, c_int64,
        _I32P, _I32P, c_int64, _I32P, c_float, _P, c_int64, _P, c_int64, _P, _P]),
    "kvc_batch_decode_run_noalloc": (c_int, [
        POINTER(KvcDecodeSchedule), _I32P, _P, c_int64, _P, _P, c_int64, c_int64, c_int64,
        _I32P, _I32P, c_int64, _I32P, c_float, _P, c_int64, _P, _P]),
    "kvc_batch_decode_append_run": (c_int, [
        POINTER(KvcDecodeSchedule), _I32P, _P, c_int64, _P, _P, c_int64, c_int64, c_int64,
        _I32P, _I32P, c_int64, _I32P, _P, c_int64, _P, c_int64, c_float, _P, c_int64, _P,
        c_int64, _P, _P]),
    "kvc_prefill_plan": (c_int, [
        c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
        POINTER(KvcPrefillSchedule), c_void_p, c_int64]),
    "kvc_batch_prefill_run": (c_int, [
        POINTER(KvcPrefillSchedule), _I32P, _P, c_int64, _P, _P, c_int64, c_int64, c_int64,
        _I32P, c_int64, c_float, _P, c_int64, _P, _P]),
    "kvc_reshape_and_cache_xpacked": (c_int, [
        _P, _P, _P, _P, _P, c_int64, c_int32, c_int32, c_int32, c_int32, c_int64, c_int64,
        c_int64, c_int64, c_int64, _P, _P]),
    "kvc_paged_attention_v1": (c_int, [
        _P, _P, c_int64, _P, _P, c_int32, c_int32, c_int32, c_int32, c_float, _I32P, c_int64,
        c_int32, _I32P, c_int32, c_int32, c_int64, c_int32, c_int64, c_int64, _P]),
    "kvc_paged_attention_v2": (c_int, [
        _P, _P, _P, _P, c_int32, _P, c_int64, _P, _P, c_int32, c_int32, c_int32, c_int32,
        c_float, _I32P, c_int64, c_int32, _I32P, c_int32, c_int32, c_int64, c_int32, c_int64,
        c_int64, _P]),
    "kvc_merge_attention_states": (c_int, [
        _P, _P, _P, _P, c_int64, c_int32, _P, _P, _P]),
    "kvc_gather_blocks": (c_int, [
        _P, _P, c_int64, c_int64, c_int64, _I32P, c_int64, _P, _I32P, _P]),
    "kvc_scatter_blocks": (c_int, [
        _P, _I32P, c_int64, _P, _P, c_int64, c_int64, c_int64, _I32P, _P]),
    "kvc_swap_out": (c_int, [
        _P, _P, c_int64, c_int64, c_int64, _I32P, c_int64, _P, c_int64, _P,
        _I32P, _P]),
    "kvc_swap_in": (c_int, [
        _P, _I32P, c_int64, _P, _P, c_int64, c_int64, c_int64, _P, c_int64,
        _I32P, _P]),
    "kvc_compute_slot_mapping": (c_int, [
        _I32P, c_int64, c_int32, c_int32, _I32P, _I32P, _I32P,
        c_int32, c_int32, c_int32, c_int32, _P, _I32P, _P]),
    "kvc_copy_page_indices": (c_int, [
        _I32P, c_int64, c_int32, _I32P, _I32P, c_int32, c_int32, _I32P, c_int64, _P]),
    "kvc_stage_from_host": (c_int, [_I32P, _I32P, c_int64, c_int64, c_int64, _P]),
    "kvc_decode_step_setup": (c_int, [
        _I32P, _I32P, POINTER(KvcDecodeStepLayout), _I32P, c_int64, c_int32, c_int32,
        _I32P, _P, c_int32, _I32P, c_int64, _P]),
}

_lock = threading.Lock()
_lib = None


class KvcError(RuntimeError):
    """A libkvc call returned a non-zero status (raised as RuntimeError, like
    the TORCH_CHECK failures of the library ops it replaces)."""

    def __init__(self, func: str, status: int, detail: str):
        self.func = func
        self.status = status
        self.detail = detail
        super().__init__(f"{func} failed with {STATUS_NAMES.get(status, status)}: {detail}")


def load(path: str | None = None) -> ctypes.CDLL:
    """Open libkvc.so once and attach the signatures of include/kvc.h."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        import torch  # noqa: F401  (bind to torch's HIP runtime, see module doc)

        p = path or LIB_PATH
        if not os.path.exists(p):
            raise RuntimeError(
                f"{p} is not built. Build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` "
                "(or gpu_offloading_amd.build.build_library()); "
                "there is no CPU fallback for the KV-cache ops.")
        if path is None:
            _check_fresh()
        lib = ctypes.CDLL(p, mode=ctypes.RTLD_LOCAL)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if path is None:
            _lib = lib
        return lib


def _check_fresh() -> None:
    """Refuse a library built from other sources than the ones beside it: its
    entry points may take other arguments than this table declares."""
    from .build import STAMP_PATH, source_hash

    try:
        with open(STAMP_PATH) as f:
            stamp = f.read().strip()
    except OSError:
        raise RuntimeError(f"{LIB_PATH} has no build stamp ({STAMP_PATH}); rebuild it with "
                           "`python -c 'import __graft_entry__ as g; g.build()'`") from None
    if stamp != source_hash():
        raise RuntimeError(f"{LIB_PATH} was built from other sources than "
                           "gpu_offloading_amd/csrc and include/kvc.h hold now; rebuild it with "
                           "`python -c 'import __graft_entry__ as g; g.build()'`")


def check(func: str, status: int) -> None:
    if status != KVC_OK:
        detail = load().kvc_last_error().decode(errors="replace")
        raise KvcError(func, status, detail)


def call(name: str, *args) -> int:
    """Call an int-status entry point and raise KvcError on failure."""
    lib = _lib if _lib is not None else load()   # no lock once loaded
    st = getattr(lib, name)(*args)
    if st != KVC_OK:
        check(name, st)
    return st


def current_stream_handle(device) -> int:
    """hipStream_t (as an int) of torch's current stream on ``device``:
    torch's raw-stream query when it has one (no Stream object is built),
    else ``torch.cuda.current_stream(device).cuda_stream``."""
    global _raw_stream
    if _raw_stream is None:
        import torch
        fn = getattr(torch._C, "_cuda_getCurrentRawStream", None)
        if fn is None:
            _raw_stream = lambda dev: torch.cuda.current_stream(dev).cuda_stream  # noqa: E731
        else:
            _raw_stream = lambda dev: fn(dev.index if dev.index is not None  # noqa: E731
                                         else torch.cuda.current_device())
    return _raw_stream(device)


_raw_stream = None
