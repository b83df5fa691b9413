"""GPU test of kvc_batch_decode_run_noalloc (the decode run whose split-K
partials live in the library's own device array) through the C ABI: on two
calls in a row, the second with a smaller batch, its output and lse equal
those of kvc_batch_decode_run with a caller workspace bit for bit (the same
kernels on the same partial layout), and match the oracle within max 2e-2 /
mean 2e-3.  A batch whose partials exceed the array is refused.  The call
is captured in a HIP graph (its first call on the device inside the capture)
and replayed, and an eager call leaves the device's free memory unchanged."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_offloading_amd import _lib, workloads
from gpu_offloading_amd.decode import BatchDecodeWithPagedKVCacheWrapper
from helpers import assert_attn_close, randn_bf16, u16
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu


def _batch(gpu, lens, seed, segs=None):
    total = sum((ln + 15) // 16 for ln in lens) + 8
    pool = orc.FifoPagePool(total, len(lens), max((ln + 15) // 16 for ln in lens),
                            free_order=workloads.randperm(total, seed))
    for s, ln in enumerate(lens):
        pool.ensure_pages(s, (ln + 15) // 16)
    kc = randn_bf16((total, 16, 8, 128), seed + 1, device=gpu)
    vc = randn_bf16((total, 16, 8, 128), seed + 2, device=gpu)
    q = randn_bf16((len(lens), 32, 128), seed + 3, device=gpu)
    indptr, lpl = orc.plan_decode(lens)
    indices = orc.page_indices(pool.block_table, range(len(lens)), indptr)
    w = BatchDecodeWithPagedKVCacheWrapper(
        torch.empty(64 << 20, dtype=torch.uint8, device=gpu), num_segments=segs)
    w.plan(torch.from_numpy(indptr), torch.from_numpy(indices).to(gpu), torch.from_numpy(lpl),
           num_qo_heads=32, num_kv_heads=8, head_dim=128, page_size=16)
    return kc, vc, q, w, (indptr, indices, lpl)


def _args(w, q, kc, vc):
    return (ctypes.byref(w._sched), w._plan_dev.data_ptr(), q.data_ptr(), q.stride(0),
            kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.shape[0],
            w._indptr.data_ptr(), w._indices.data_ptr(), w._num_indices, w._lpl.data_ptr(),
            ctypes.c_float(w._sm_scale))


def _run_both(gpu, lens, seed, segs=None):
    kc, vc, q, w, (indptr, indices, lpl) = _batch(gpu, lens, seed, segs)
    sched = w._sched
    assert sched.max_partitions > 1 and sched.workspace_bytes > 0   # partials are used
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    B = len(lens)
    out_ws = torch.empty(B, 32, 128, dtype=torch.bfloat16, device=gpu)
    lse_ws = torch.empty(B, 32, dtype=torch.float32, device=gpu)
    ws = w._workspace
    st = lib.kvc_batch_decode_run(*_args(w, q, kc, vc), ws.data_ptr(), ws.numel(),
                                  out_ws.data_ptr(), out_ws.stride(0), lse_ws.data_ptr(), stream)
    assert st == 0, lib.kvc_last_error()
    out_na = torch.full_like(out_ws, float("nan"))
    lse_na = torch.full_like(lse_ws, float("nan"))
    st = lib.kvc_batch_decode_run_noalloc(*_args(w, q, kc, vc), out_na.data_ptr(),
                                          out_na.stride(0), lse_na.data_ptr(), stream)
    assert st == 0, lib.kvc_last_error()
    torch.cuda.synchronize()
    assert torch.equal(out_na, out_ws) and torch.equal(lse_na, lse_ws)
    ref, ref_lse = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
    assert_attn_close(out_na.float().cpu().numpy(), ref)
    assert np.abs(lse_na.cpu().numpy() - ref_lse).max() < 2e-3
    return sched


def test_noalloc_decode_captured_in_a_graph_matches_eager(gpu):
    """What the entry point is for: a caller that cannot allocate captures it
    in a HIP graph.  Only a workspace run (which loads the kernels) precedes
    the capture, so the first allocation-free call on this device -- the
    lookup of its array's address -- happens inside the capture.  Three
    replays with new q (eager work and synchronisations between them) each
    equal the eager workspace run bit for bit; an eager call then leaves the
    device's free memory unchanged (hipMemGetInfo)."""
    print("noalloc: capture of the first call on the device", flush=True)
    lens = [3000, 17, 1, 900, 4096, 256, 33]
    kc, vc, q, w, _ = _batch(gpu, lens, 60, segs=97)
    assert w._sched.max_partitions > 1
    lib = _lib.load()
    B = len(lens)
    ws = w._workspace
    q_in = torch.zeros_like(q)
    out_g = torch.empty(B, 32, 128, dtype=torch.bfloat16, device=gpu)
    lse_g = torch.empty(B, 32, dtype=torch.float32, device=gpu)
    out_ws, lse_ws = torch.empty_like(out_g), torch.empty_like(lse_g)

    def workspace_run(qq, stream):
        st = lib.kvc_batch_decode_run(*_args(w, qq, kc, vc), ws.data_ptr(), ws.numel(),
                                      out_ws.data_ptr(), out_ws.stride(0), lse_ws.data_ptr(),
                                      stream)
        assert st == 0, lib.kvc_last_error()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        workspace_run(q_in, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = lib.kvc_batch_decode_run_noalloc(*_args(w, q_in, kc, vc), out_g.data_ptr(),
                                              out_g.stride(0), lse_g.data_ptr(),
                                              torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.kvc_last_error()
    g = torch.Generator(device=gpu).manual_seed(61)
    for rep in range(3):
        q_new = torch.randn(q.shape, generator=g, device=gpu).to(torch.bfloat16)
        q_in.copy_(q_new)
        graph.replay()
        got, got_lse = out_g.clone(), lse_g.clone()
        torch.cuda.synchronize()
        workspace_run(q_new, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        assert torch.equal(got, out_ws) and torch.equal(got_lse, lse_ws), rep
    free0 = torch.cuda.mem_get_info()[0]
    st = lib.kvc_batch_decode_run_noalloc(*_args(w, q_in, kc, vc), out_g.data_ptr(),
                                          out_g.stride(0), lse_g.data_ptr(),
                                          torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.kvc_last_error()
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    del graph


def test_noalloc_decode_matches_the_workspace_run_twice(gpu):
    print("noalloc: first call (cfg2-shaped batch of 64)", flush=True)
    lens = [ln + 1 for ln in workloads.config2(seed=0).seq_lens]
    big = _run_both(gpu, lens, 30)
    print("noalloc: second call (smaller batch of 7, more pieces each)", flush=True)
    small = _run_both(gpu, [3000, 17, 1, 900, 4096, 256, 33], 40, segs=97)
    assert small.batch < big.batch


def test_noalloc_decode_refuses_partials_beyond_its_array(gpu):
    print("noalloc: oversized schedule refused", flush=True)
    lens = [320] * 64                      # 20 one-page pieces per request: 21 MB of partials
    kc, vc, q, w, _ = _batch(gpu, lens, 50, segs=1280)
    assert w._sched.workspace_bytes > 16 << 20
    lib = _lib.load()
    out = torch.empty(64, 32, 128, dtype=torch.bfloat16, device=gpu)
    st = lib.kvc_batch_decode_run_noalloc(*_args(w, q, kc, vc), out.data_ptr(), out.stride(0),
                                          None, torch.cuda.current_stream().cuda_stream)
    assert st == _lib.KVC_ERR_WORKSPACE
    assert b"allocation-free" in lib.kvc_last_error()
