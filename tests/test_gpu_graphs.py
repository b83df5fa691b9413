"""HIP-graph capture of the path's launches (the engine captures the KV
append inside its stage-1 CUDA graph, moe_engine.py:2312-2352): the captured
append and a captured decode run (within one plan) are replayed several
times, with new inputs copied into the static buffers and eager work and
synchronisations between replays; every replay equals the eager result."""
import pytest
import torch

from gpu_offloading_amd import ops, workloads
from gpu_offloading_amd.decode import BatchDecodeWithPagedKVCacheWrapper
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu


def test_captured_append_and_decode_replays_match_eager(gpu):
    g = torch.Generator(device=gpu).manual_seed(95)
    hkv, hq, nb = 8, 32, 64
    lens = [40, 17, 200]
    kv = torch.randn(nb, 2, 16, hkv, 128, generator=g, device=gpu).to(torch.bfloat16)
    kc, vc = kv[:, 0], kv[:, 1]
    pool = orc.FifoPagePool(nb, 3, 16, free_order=workloads.randperm(nb, 96))
    for s, ln in enumerate(lens):
        pool.ensure_pages(s, (ln + 15) // 16)
    bt = pool.block_table
    slots = torch.tensor([int(bt[s, (ln - 1) // 16]) * 16 + (ln - 1) % 16
                          for s, ln in enumerate(lens)], dtype=torch.int64, device=gpu)
    indptr, lpl = orc.plan_decode(lens)
    idx = torch.from_numpy(orc.page_indices(bt, range(3), indptr)).to(gpu)
    w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(1 << 24, dtype=torch.uint8, device=gpu))
    w.plan(torch.from_numpy(indptr), idx, torch.from_numpy(lpl), num_qo_heads=hq,
           num_kv_heads=hkv, head_dim=128, page_size=16)
    k_in = torch.zeros(3, hkv, 128, dtype=torch.bfloat16, device=gpu)
    v_in = torch.zeros_like(k_in)
    q_in = torch.zeros(3, hq, 128, dtype=torch.bfloat16, device=gpu)
    out = torch.empty_like(q_in)
    # warm up on a side stream, then capture append + decode
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.reshape_and_cache_flash(k_in, v_in, kc, vc, slots)
        w.run(q_in, (kc, vc), out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.reshape_and_cache_flash(k_in, v_in, kc, vc, slots)
        w.run(q_in, (kc, vc), out=out)
    for rep in range(4):
        k_new = torch.randn(3, hkv, 128, generator=g, device=gpu).to(torch.bfloat16)
        v_new = torch.randn(3, hkv, 128, generator=g, device=gpu).to(torch.bfloat16)
        q_new = torch.randn(3, hq, 128, generator=g, device=gpu).to(torch.bfloat16)
        k_in.copy_(k_new)
        v_in.copy_(v_new)
        q_in.copy_(q_new)
        graph.replay()
        got_out = out.clone()
        got_kv = kv.clone()
        torch.cuda.synchronize()
        # eager on a copy of the pre-replay state gives the same bytes
        ops.reshape_and_cache_flash(k_new, v_new, kc, vc, slots)
        want_out = w.run(q_new, (kc, vc))
        torch.cuda.synchronize()
        assert torch.equal(got_kv, kv), rep
        assert torch.equal(got_out, want_out), rep


def test_graph_mode_wrappers_are_refused(gpu):
    from gpu_offloading_amd.prefill import BatchPrefillWithPagedKVCacheWrapper

    ws = torch.empty(1 << 20, dtype=torch.uint8, device=gpu)
    with pytest.raises(RuntimeError, match="use_cuda_graph"):
        BatchDecodeWithPagedKVCacheWrapper(ws, "NHD", use_cuda_graph=True)
    with pytest.raises(RuntimeError, match="use_cuda_graph"):
        BatchPrefillWithPagedKVCacheWrapper(ws, "NHD", use_cuda_graph=True)
