"""The C ABI (include/kvc.h) on the CPU: the library loads, exports every
declared entry point, the ctypes table matches the header, and the host-only
entry points (version, status strings, decode planning, argument checks) work
without a GPU.  No kernel is launched here."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from gpu_offloading_amd import _lib
from gpu_offloading_amd.build import INCLUDE, LIB_PATH, build_library

HEADER = os.path.join(INCLUDE, "kvc.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB_PATH):
        build_library()
    return _lib.load()


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvc_\w+)\s*\(", text)))


def test_header_and_ctypes_table_agree():
    assert header_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (kvc_\w+)", out))
    missing = set(header_functions()) - exported
    assert not missing, f"not exported: {sorted(missing)}"
    for name in header_functions():
        assert getattr(lib, name) is not None


def test_argument_counts_match_header():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    for name, (_, argtypes) in _lib.SIGNATURES.items():
        m = re.search(rf"\b{name}\s*\((.*?)\)\s*;", text, flags=re.S)
        assert m, name
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(argtypes), (name, len(params), len(argtypes))


def test_version_and_status_strings(lib):
    assert lib.kvc_version() >= 100
    assert lib.kvc_status_string(0) == b"ok"
    assert b"workspace" in lib.kvc_status_string(4)


def test_decode_plan_is_host_only_and_splits_partitions(lib):
    lens = np.array([1, 16, 17, 4096, 0], np.int64)
    pages = (lens + 15) // 16
    indptr = np.zeros(len(lens) + 1, np.int32)
    np.cumsum(pages, out=indptr[1:])
    sched = _lib.KvcDecodeSchedule()
    st = lib.kvc_decode_plan(indptr.ctypes.data, len(lens), 32, 8, 128, 16, 8, 256,
                             ctypes.byref(sched))
    assert st == 0
    assert sched.pages_per_partition == 8
    assert sched.max_partitions == 32          # 256 pages / 8
    assert sched.total_pages == int(pages.sum())
    assert sched.num_empty == 1
    assert sched.workspace_bytes == lib.kvc_decode_workspace_bytes(len(lens), 32, 128, 32)
    # rounding of the hint to a multiple of 4 and the upper clamp
    lib.kvc_decode_plan(indptr.ctypes.data, len(lens), 32, 8, 128, 16, 5, 256, ctypes.byref(sched))
    assert sched.pages_per_partition == 8
    lib.kvc_decode_plan(indptr.ctypes.data, len(lens), 32, 8, 128, 16, 100000, 256,
                        ctypes.byref(sched))
    assert sched.pages_per_partition == 256 and sched.max_partitions == 1


def test_decode_plan_rejects_bad_shapes(lib):
    indptr = np.array([0, 3], np.int32)
    sched = _lib.KvcDecodeSchedule()
    assert lib.kvc_decode_plan(indptr.ctypes.data, 1, 12, 8, 128, 16, 0, 256, ctypes.byref(sched)) == 1
    assert b"multiple" in lib.kvc_last_error()
    assert lib.kvc_decode_plan(indptr.ctypes.data, 1, 32, 8, 96, 16, 0, 256, ctypes.byref(sched)) == 2
    assert lib.kvc_decode_plan(indptr.ctypes.data, 1, 32, 8, 128, 32, 0, 256, ctypes.byref(sched)) == 2
    bad = np.array([0, 5, 3], np.int32)
    assert lib.kvc_decode_plan(bad.ctypes.data, 2, 32, 8, 128, 16, 0, 256, ctypes.byref(sched)) == 1
    assert b"non-decreasing" in lib.kvc_last_error()


def test_entry_points_validate_before_touching_the_gpu(lib):
    # Zero-sized calls succeed and null pointers are rejected, all on the host.
    assert lib.kvc_reshape_and_cache_flash(None, None, None, None, None, 0, 8, 128, 16, 4, 2,
                                           1024, 1024, 16384, 1024, None, None) == 0
    assert lib.kvc_reshape_and_cache_flash(None, None, None, None, None, 5, 8, 128, 16, 4, 2,
                                           1024, 1024, 16384, 1024, None, None) == 1
    assert b"null pointer" in lib.kvc_last_error()
    assert lib.kvc_gather_blocks(None, None, 65536, 65536, 8, None, 0, None, None, None) == 0
    assert lib.kvc_gather_blocks(None, None, 65536, 65536, 8, None, 3, None, None, None) == 1
    assert lib.kvc_swap_out(None, None, 65536, 65536, 8, None, -1, None, 0, None, None, None) == 1
    assert lib.kvc_compute_slot_mapping(None, 0, 1, 1, None, None, None, 0, 0, 0, 16,
                                        None, None, None) == 0
    assert lib.kvc_copy_page_indices(None, 0, 1, None, None, 0, 1, None, None) == 0
    assert lib.kvc_merge_attention_states(None, None, None, None, 0, 128, None, None, None) == 0
