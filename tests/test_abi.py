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


def _plan(lib, lens, hq=32, hkv=8, d=128, hint=0, cus=256):
    lens = np.asarray(lens, np.int64)
    pages = (lens + 15) // 16
    indptr = np.zeros(len(lens) + 1, np.int32)
    np.cumsum(pages, out=indptr[1:])
    lpl = np.where((lens % 16 == 0) & (lens > 0), 16, lens % 16).astype(np.int32)
    sched = _lib.KvcDecodeSchedule()
    cap = 16
    for _ in range(2):   # the first call reports the capacity it needs
        img = np.zeros(cap, np.int32)
        st = lib.kvc_decode_plan(indptr.ctypes.data, lpl.ctypes.data, len(lens), hq, hkv, d,
                                 16, hint, cus, ctypes.byref(sched), img.ctypes.data, cap)
        if st == 4:
            assert sched.plan_ints > cap
            cap = sched.plan_ints
    assert st == 0, lib.kvc_last_error()
    assert sched.plan_ints == lib.kvc_decode_plan_ints(len(lens), sched.num_segments)
    return indptr, sched, img, lpl


def _check_small_plan_image(indptr, sched, img, lpl):
    """Small-batch plans: one segment and one piece per request (empty ones
    included), piece b = request b's whole page range, no partials."""
    B = sched.batch
    assert sched.small_batch == 1 and sched.num_segments == B and sched.num_pieces == B
    assert sched.heads_per_group == 1 and sched.num_head_groups == sched.num_kv_heads
    assert sched.max_partitions == 1 and sched.workspace_bytes == 0
    segs = img[:4 * B].reshape(-1, 4)
    rec = img[sched.pieces_offset:sched.pieces_offset + 8 * B].reshape(-1, 8)
    nparts = img[sched.nparts_offset:sched.nparts_offset + B]
    pages = np.diff(indptr)
    assert (segs[:, 0] == np.arange(B)).all() and (segs[:, 1] == np.arange(1, B + 1)).all()
    assert (segs[:, 2] == indptr[:-1]).all() and (segs[:, 3] == pages).all()
    assert (rec[:, 0] == np.arange(B)).all() and (rec[:, 3] == -1).all()
    assert (rec[:, 1] == indptr[:-1]).all() and (rec[:, 2] == indptr[1:]).all()
    assert (rec[:, 4] == indptr[1:] - 1).all() and (rec[:, 5] == lpl).all()
    assert (nparts == (pages > 0)).all()
    assert pages.max() <= 16


def _segment_costs(indptr, segs):
    """Planner cost of each segment [g0, g1): 8 per page plus 9 per request
    start in [g0, g1) (the first request's start excluded)."""
    starts = [int(indptr[b]) for b in range(1, len(indptr) - 1)
              if indptr[b + 1] > indptr[b] and indptr[b] > 0]
    return [8 * int(n) + 9 * sum(1 for x in starts if g0 <= x < g0 + n) for _, _, g0, n in segs]


def _check_plan_image(indptr, sched, img, lpl):
    """Segments are contiguous, at least one and at most 128 pages, and equal
    in cost (8 per page, 9 per switch to another request) to within the cost
    of one step, or equal in pages to within one when balanced costs would
    exceed 128 pages; their pieces tile every request's pages exactly once,
    numbered 0..n-1 per request (-1 when a request is a single piece), each
    carrying its request's last slot and last-page length."""
    if sched.small_batch:
        return _check_small_plan_image(indptr, sched, img, lpl)
    S = sched.num_segments
    segs = img[:4 * S].reshape(-1, 4)
    rec = img[sched.pieces_offset:sched.pieces_offset + 8 * sched.num_pieces].reshape(-1, 8)
    pieces = rec[:, :4]
    nparts = img[sched.nparts_offset:sched.nparts_offset + sched.batch]
    total = int(indptr[-1])
    assert sched.total_pages == total
    assert segs[0, 0] == 0 and segs[-1, 1] == sched.num_pieces
    assert (segs[1:, 0] == segs[:-1, 1]).all()
    lengths = []
    for s in range(S):
        ps = pieces[segs[s, 0]:segs[s, 1]]
        assert len(ps) >= 1
        assert (ps[1:, 1] == ps[:-1, 2]).all()                 # contiguous slots
        assert ps[0, 1] == (0 if s == 0 else segs[s - 1, 2] + segs[s - 1, 3])
        assert segs[s, 2] == ps[0, 1] and segs[s, 3] == ps[-1, 2] - ps[0, 1]
        lengths.append(ps[-1, 2] - ps[0, 1])
    assert segs[-1, 2] + segs[-1, 3] == total
    assert min(lengths) >= 1 and max(lengths) <= 128
    costs = _segment_costs(indptr, segs)
    assert max(costs) - min(costs) < 2 * (8 + 9) or max(lengths) - min(lengths) <= 1
    assert (rec[:, 4] == indptr[rec[:, 0] + 1] - 1).all()
    assert (rec[:, 5] == lpl[rec[:, 0]]).all()
    for b in range(sched.batch):
        mine = pieces[pieces[:, 0] == b]
        assert len(mine) == nparts[b]
        if len(mine) == 0:
            assert indptr[b + 1] == indptr[b]
            continue
        assert mine[0, 1] == indptr[b] and mine[-1, 2] == indptr[b + 1]
        assert (mine[1:, 1] == mine[:-1, 2]).all()
        if len(mine) == 1:
            assert mine[0, 3] == -1
        else:
            assert mine[:, 3].tolist() == list(range(len(mine)))
    assert sched.max_partitions == max(1, int(nparts.max()))
    # append_pieces: over segments, the most leading pieces up to the last
    # one that ends its request (the fused append stages rows by this index)
    want = 0
    for s in range(S):
        ps = rec[segs[s, 0]:segs[s, 1]]
        ends = [i + 1 for i, pc in enumerate(ps) if pc[2] == pc[4] + 1]
        want = max([want] + ends)
    assert sched.append_pieces == want


def test_decode_plan_is_host_only_and_balanced(lib):
    lens = [1, 16, 17, 4096, 0, 300, 2049, 33]
    indptr, sched, img, lpl = _plan(lib, lens, hint=40)
    # 8 KV heads of head_dim 128 stream together (one workgroup per segment)
    assert sched.num_segments == 40 and sched.num_head_groups == 1
    assert sched.heads_per_group == 8
    assert sched.num_empty == 1
    _check_plan_image(indptr, sched, img, lpl)
    assert sched.workspace_bytes == lib.kvc_decode_workspace_bytes(
        len(lens), 32, 128, sched.max_partitions)
    # default: one segment per resident workgroup (256 CUs x 1 of 8 heads)
    indptr, sched, img, lpl = _plan(lib, [3000] * 64)
    assert sched.num_segments == 256
    _check_plan_image(indptr, sched, img, lpl)
    assert sched.append_pieces == 1          # a segment holds at most one request end
    # many short requests: several ends per segment (the fused append falls back)
    indptr, sched, img, lpl = _plan(lib, [3] * 1500)
    _check_plan_image(indptr, sched, img, lpl)
    assert sched.append_pieces > 4
    # KV heads that do not divide by 8 stream one per workgroup
    indptr, sched, img, lpl = _plan(lib, [3000] * 64, hq=24, hkv=6)
    assert sched.heads_per_group == 1 and sched.num_head_groups == 6
    _check_plan_image(indptr, sched, img, lpl)
    # head_dim 64 / 256 kernels group 4 heads
    indptr, sched, img, lpl = _plan(lib, [3000] * 8, hq=32, hkv=8, d=64)
    assert sched.heads_per_group == 4 and sched.num_head_groups == 2
    _check_plan_image(indptr, sched, img, lpl)
    # segments never exceed 128 pages, never hold less than one page
    indptr, sched, img, lpl = _plan(lib, [16 * 5000], hint=2)
    assert sched.num_segments == 40
    _check_plan_image(indptr, sched, img, lpl)
    # past 128 pages per resident slot, whole rounds of slots: 40000 pages
    # need 313 segments, rounded up to 2 x 256
    indptr, sched, img, lpl = _plan(lib, [16 * 20000] * 2)
    assert sched.num_segments == 512
    _check_plan_image(indptr, sched, img, lpl)
    indptr, sched, img, lpl = _plan(lib, [16 * 20000] * 2, cus=100)
    assert sched.num_segments == 400
    _check_plan_image(indptr, sched, img, lpl)
    indptr, sched, img, lpl = _plan(lib, [40, 1], hint=1000)
    assert sched.num_segments == 4
    _check_plan_image(indptr, sched, img, lpl)


@pytest.mark.parametrize("lens", [[0, 5], [10, 10, 10, 10, 0], [0, 0]])
def test_decode_plan_empty_requests_without_splits(lib, lens):
    """Empty requests next to requests of one piece each: no partials exist
    (max_partitions 1, workspace 0); the run's merge launch then only zeroes
    the empty requests and must not read partials."""
    indptr, sched, img, lpl = _plan(lib, lens)
    assert sched.max_partitions == 1
    assert sched.num_empty == lens.count(0)
    assert sched.workspace_bytes == 0
    assert lib.kvc_decode_workspace_bytes(len(lens), 32, 128, 1) == 0
    if sum(lens) == 0:
        assert sched.num_segments == 0 and sched.num_pieces == 0
    else:
        _check_plan_image(indptr, sched, img, lpl)
        rec = img[sched.pieces_offset:sched.pieces_offset + 8 * sched.num_pieces].reshape(-1, 8)
        assert (rec[:, 3] == -1).all()          # every piece is written directly
    nparts = img[sched.nparts_offset:sched.nparts_offset + sched.batch]
    assert nparts.tolist() == [0 if ln == 0 else 1 for ln in lens]


def test_decode_run_refuses_split_plan_without_partials(lib):
    """A plan that splits a request needs the partials workspace: the run is
    refused on the host (no launch) when it is absent or too small."""
    indptr, sched, img, lpl = _plan(lib, [0, 1000, 3], hint=8)
    assert sched.max_partitions > 1 and sched.workspace_bytes > 0
    fake = 1 << 20     # aligned, never dereferenced: the call fails before any launch
    for ws, nbytes in ((None, 0), (fake, sched.workspace_bytes - 256)):
        st = lib.kvc_batch_decode_run(ctypes.byref(sched), fake, fake, 4096, fake, fake,
                                      2 * 16 * 1024, 1024, 100, fake, fake, 100, fake,
                                      0.088, ws, nbytes, fake, 4096, None, None)
        assert st == 4, lib.kvc_last_error()
        assert b"workspace" in lib.kvc_last_error()


def test_small_batch_plans_are_chosen_only_where_segments_would_split(lib):
    """Per-request workgroups replace the equal segments when every request
    fits in 16 pages and the segments would cut one (batch 1 at the
    reference's 128-token context: 9 one-page segments and a merge
    otherwise); never with a forced segment count or head_dim != 128."""
    for lens in ([129], [129] * 4, [0, 129, 3], [256] * 40, [1, 2, 200]):
        indptr, sched, img, lpl = _plan(lib, lens)
        assert sched.small_batch == 1, lens
        _check_plan_image(indptr, sched, img, lpl)
        assert sched.num_empty == lens.count(0)
    for lens, kw in (([257], {}),                      # 17 pages: too long
                     ([3000] * 64, {}),                 # the bench's shape
                     ([16] * 300, {}),                  # one page each: nothing to split
                     ([129], {"hint": 9}),              # forced segments
                     ([129], {"d": 64, "hq": 32, "hkv": 8})):
        indptr, sched, img, lpl = _plan(lib, lens, **kw)
        assert sched.small_batch == 0, (lens, kw)
        _check_plan_image(indptr, sched, img, lpl)


def test_noalloc_run_refuses_partials_beyond_its_array_on_the_host(lib):
    """kvc_batch_decode_run_noalloc checks the schedule's partials against
    its fixed device array before touching the GPU (no device here)."""
    indptr, sched, img, lpl = _plan(lib, [320] * 64, hint=1280)
    assert sched.workspace_bytes > 16 << 20
    fake = 1 << 20
    st = lib.kvc_batch_decode_run_noalloc(ctypes.byref(sched), fake, fake, 4096, fake, fake,
                                          2 * 16 * 1024, 1024, 2000, fake, fake, 1280, fake,
                                          0.088, fake, 4096, None, None)
    assert st == 4
    assert b"allocation-free" in lib.kvc_last_error()
    empty = _lib.KvcDecodeSchedule()            # batch 0: nothing to do
    assert lib.kvc_batch_decode_run_noalloc(ctypes.byref(empty), None, None, 0, None, None,
                                            0, 0, 0, None, None, 0, None, 0.1, None, 0,
                                            None, None) == 0


@pytest.mark.parametrize("lens, hint, starts", [
    # four 10-page requests, four segments: cut on the request boundaries
    # (no request split, so no partials at all)
    ([160] * 4, 4, [0, 10, 20, 30]),
    # pages 6, 30, 4: cost 8 x 40 + 9 x 2 switches = 338; the cut at page 20
    # gives 8 x 20 + 9 (the switch at page 6) = 169 on each side
    ([96, 480, 64], 2, [0, 20]),
    # pages 2, 2, 2, 2, 32: cost 320 + 4 x 9 = 356, half 178; F(17) = 136 +
    # 36 = 172 and F(18) = 144 + 36 = 180, so the cut is page 18, two pages
    # before the equal-page cut: segment 0 (18 pages, 4 switches) costs 180,
    # segment 1 (22 pages) 176
    ([32, 32, 32, 32, 512], 2, [0, 18]),
])
def test_decode_plan_cuts_balance_pages_and_switches(lib, lens, hint, starts):
    """Segment cuts, worked by hand: a page costs 8, a switch to another
    request inside a segment 9 more; each cut goes where the cost of the pages
    before it is nearest to its share of the total."""
    indptr, sched, img, lpl = _plan(lib, lens, hint=hint)
    _check_plan_image(indptr, sched, img, lpl)
    segs = img[:4 * sched.num_segments].reshape(-1, 4)
    assert segs[:, 2].tolist() == starts
    if starts == [0, 10, 20, 30]:
        assert sched.max_partitions == 1 and sched.workspace_bytes == 0


def test_decode_plan_random_batches(lib):
    rng = np.random.default_rng(0)
    for trial in range(30):
        lens = rng.integers(0, 3000, rng.integers(1, 80)).tolist()
        hkv = int(rng.choice([1, 4, 8, 16]))
        hint = int(rng.choice([0, 1, 7, 64, 333]))
        indptr, sched, img, lpl = _plan(lib, lens, hq=hkv * 4, hkv=hkv, hint=hint,
                                   cus=int(rng.integers(1, 300)))
        if indptr[-1] == 0:
            assert sched.num_segments == 0
            continue
        _check_plan_image(indptr, sched, img, lpl)


def test_decode_plan_reports_the_needed_capacity(lib):
    indptr = np.array([0, 100, 100, 300], np.int32)
    lpl = np.array([16, 0, 16], np.int32)
    sched = _lib.KvcDecodeSchedule()
    small = np.zeros(4, np.int32)
    st = lib.kvc_decode_plan(indptr.ctypes.data, lpl.ctypes.data, 3, 32, 8, 128, 16, 50, 256,
                             ctypes.byref(sched), small.ctypes.data, 4)
    assert st == 4 and sched.plan_ints == lib.kvc_decode_plan_ints(3, 50)
    assert b"plan buffer too small" in lib.kvc_last_error()


def test_decode_plan_rejects_bad_shapes(lib):
    indptr = np.array([0, 3], np.int32)
    sched = _lib.KvcDecodeSchedule()
    img = np.zeros(4096, np.int32)

    lpl = np.full(4, 16, np.int32)

    def plan(hq, hkv, d, ps, ip=indptr, batch=1):
        return lib.kvc_decode_plan(ip.ctypes.data, lpl.ctypes.data, batch, hq, hkv, d, ps, 0, 256,
                                   ctypes.byref(sched), img.ctypes.data, img.size)

    assert plan(12, 8, 128, 16) == 1
    assert b"multiple" in lib.kvc_last_error()
    assert plan(32, 8, 96, 16) == 2
    assert plan(32, 8, 128, 32) == 2
    assert plan(32, 8, 128, 16, np.array([0, 5, 3], np.int32), 2) == 1
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
    assert lib.kvc_copy_page_indices(None, 0, 1, None, None, 0, 1, None, 0, None) == 0
    assert lib.kvc_copy_page_indices(None, 0, 1, None, None, 0, 1, None, -1, None) == 1
    assert lib.kvc_gather_kv(None, None, None, 0, 1, None, None, 0, 0, 8, 128, 16, 4, 2,
                             16384, 1024, None, None, 1024, 0, None, None) == 0
    assert lib.kvc_gather_kv(None, None, None, 0, 1, None, None, 1, 5, 8, 128, 16, 4, 2,
                             16384, 1024, None, None, 1024, -1, None, None) == 1
    assert lib.kvc_merge_attention_states(None, None, None, None, 0, 128, None, None, None) == 0


def _prefill_plan(lib, q_lens, kv_lens, hq=32, hkv=8, causal=1, cap=None):
    """kvc_prefill_plan; returns (status, schedule, workgroup table [W, 2],
    unit records [U, 8], qo_indptr, kv_indptr)."""
    qo = np.zeros(len(q_lens) + 1, np.int32)
    np.cumsum(q_lens, out=qo[1:])
    pages = [(k + 15) // 16 for k in kv_lens]
    kvi = np.zeros(len(kv_lens) + 1, np.int32)
    np.cumsum(pages, out=kvi[1:])
    lpl = np.array([(k % 16 or 16) if k else 0 for k in kv_lens], np.int32)
    sched = _lib.KvcPrefillSchedule()
    img = np.zeros(cap if cap is not None else 8 * 4096, np.int32)
    st = lib.kvc_prefill_plan(qo.ctypes.data, kvi.ctypes.data, lpl.ctypes.data, len(q_lens),
                              hq, hkv, 128, 16, causal, ctypes.byref(sched), img.ctypes.data,
                              img.size)
    w = min(256, sched.num_items * hkv)
    table = (2 * w + 3) // 4 * 4
    if st != 0:
        return st, sched, None, None, qo, kvi
    assert sched.plan_ints == table + 8 * sched.num_items * hkv
    return st, sched, img[:2 * w].reshape(-1, 2), img[table:sched.plan_ints].reshape(-1, 8), qo, kvi


def test_prefill_plan_tiles_every_query_once_per_head(lib):
    q_lens, kv_lens = [1, 17, 40, 64, 130, 0, 33], [1, 40, 40, 300, 130, 12, 1000]
    hkv = 8
    st, sched, wg, rec, qo, kvi = _prefill_plan(lib, q_lens, kv_lens, hkv=hkv)
    assert st == 0, lib.kvc_last_error()
    T = sched.tile_tokens                                         # 256 query rows / group 4
    assert T == 64 and sched.total_q == sum(q_lens)
    n = sched.num_items
    assert n == sum((q + T - 1) // T for q in q_lens) and len(rec) == n * hkv
    # the table covers the records once, in order
    assert wg[0, 0] == 0 and (wg[1:, 0] == np.cumsum(wg[:-1, 1])).all() and wg[:, 1].sum() == len(rec)
    for b, (ql, kl) in enumerate(zip(q_lens, kv_lens)):
        mine = rec[(rec[:, 4] == qo[b]) & (rec[:, 5] == kvi[b]) & (rec[:, 2] == ql)]
        for h in range(hkv):
            assert sorted(mine[mine[:, 0] == h][:, 1].tolist()) == list(range(0, ql, T))
        for r in mine:
            assert (r[2], r[3], r[4], r[5], r[7]) == (ql, kl, qo[b], kvi[b], kvi[b + 1] - kvi[b])
            last = min(r[1] + T, ql) - 1
            keys = max(0, min(last + kl - ql + 1, kl))
            assert r[6] == (keys + 63) // 64
    assert sched.max_key_tiles == rec[:, 6].max()
    # non-causal: every tile visits the whole cache
    st, sched, wg, rec, _, _ = _prefill_plan(lib, q_lens, kv_lens, causal=0)
    assert st == 0
    assert all(r[6] == (r[3] + 63) // 64 for r in rec)
    # group 8 packs 32 tokens x 8 heads per tile
    st, sched, wg, rec, _, _ = _prefill_plan(lib, [100], [100], hq=16, hkv=2)
    assert st == 0 and sched.tile_tokens == 32 and sched.num_items == 4 and len(wg) == 8


def test_prefill_plan_balances_the_workgroups(lib):
    """256 persistent workgroups, unit costs key tiles + 2: within each XCD's
    32 workgroups the loads differ by at most one unit's cost (list
    scheduling), and the workgroups of one XCD run one request's units."""
    q_lens, kv_lens = [2048] * 8, [4096] * 8
    st, sched, wg, rec, qo, _ = _prefill_plan(lib, q_lens, kv_lens)
    assert st == 0 and len(wg) == 256 and len(rec) == 256 * 8
    cost = rec[:, 6] + 2
    loads = np.array([cost[f:f + c].sum() for f, c in wg])
    for x in range(8):
        mine = loads[x::8]
        assert mine.max() - mine.min() <= cost.max(), (x, mine.min(), mine.max())
        reqs = {int(r[4]) for f, c in wg[x::8] for r in rec[f:f + c]}
        assert reqs == {int(qo[x])}, (x, reqs)
    # fewer units than workgroups: one unit each
    st, sched, wg, rec, _, _ = _prefill_plan(lib, [100], [300])
    assert st == 0 and len(wg) == len(rec) == 2 * 8 and (wg[:, 1] == 1).all()


def test_prefill_plan_reports_capacity_and_rejects_bad_input(lib):
    st, sched, _, _, _, _ = _prefill_plan(lib, [100, 40], [100, 40], cap=8)
    assert st == 4 and sched.plan_ints == 48 + 8 * 3 * 8          # table + 24 unit records
    assert b"plan buffer too small" in lib.kvc_last_error()
    st, *_ = _prefill_plan(lib, [10], [10], hq=24, hkv=8)
    assert st == 2                                                 # group 3
    qo = np.array([0, 5, 3], np.int32)
    kvi = np.array([0, 1, 2], np.int32)
    lpl = np.array([5, 3], np.int32)
    sched = _lib.KvcPrefillSchedule()
    img = np.zeros(64, np.int32)
    assert lib.kvc_prefill_plan(qo.ctypes.data, kvi.ctypes.data, lpl.ctypes.data, 2, 32, 8, 128,
                                16, 1, ctypes.byref(sched), img.ctypes.data, 64) == 1
    assert b"non-decreasing" in lib.kvc_last_error()
    # zero items: the run is a no-op even with null pointers
    st, sched, _, _, _, _ = _prefill_plan(lib, [0], [16])
    assert st == 0 and sched.num_items == 0
    assert lib.kvc_batch_prefill_run(ctypes.byref(sched), None, None, 4096, None, None, 16384,
                                     1024, 1, None, 0, 0.1, None, 4096, None, None) == 0


def test_a_library_built_from_other_sources_is_refused(tmp_path, monkeypatch):
    """The build stamps libkvc.so with a hash of its sources; loading checks it,
    so a library whose entry points may differ from this ctypes table is never
    called."""
    from gpu_offloading_amd import build

    assert open(build.STAMP_PATH).read().strip() == build.source_hash()
    _lib._check_fresh()                                     # the current build passes
    stale = tmp_path / "stamp"
    stale.write_text("0" * 64 + "\n")
    monkeypatch.setattr(build, "STAMP_PATH", str(stale))
    with pytest.raises(RuntimeError, match="other sources"):
        _lib._check_fresh()
    monkeypatch.setattr(build, "STAMP_PATH", str(tmp_path / "missing"))
    with pytest.raises(RuntimeError, match="no build stamp"):
        _lib._check_fresh()


def test_struct_layouts_match_header(tmp_path):
    """The ctypes mirrors of the header's structs have the C layout: every
    field's offset and each struct's size, from a program compiled against
    include/kvc.h with the host C compiler."""
    mirrors = {"kvc_decode_schedule": _lib.KvcDecodeSchedule,
               "kvc_prefill_schedule": _lib.KvcPrefillSchedule,
               "kvc_decode_step_layout": _lib.KvcDecodeStepLayout}
    lines = ['#include <stddef.h>', '#include <stdio.h>', '#include "kvc.h"', 'int main(void) {']
    for name, cls in mirrors.items():
        lines.append(f'  printf("{name} size %zu\\n", sizeof({name}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("{name} {field} %zu\\n", offsetof({name}, {field}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-I", INCLUDE, str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True,
                               check=True).stdout.splitlines():
        struct, field, value = line.split()
        got[(struct, field)] = int(value)
    for name, cls in mirrors.items():
        assert got[(name, "size")] == ctypes.sizeof(cls), name
        for field, _ in cls._fields_:
            assert got[(name, field)] == getattr(cls, field).offset, (name, field)
