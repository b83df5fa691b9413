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


def test_decode_step_graph_replays_across_planned_steps(gpu):
    """A whole decode step of a PagedKVCache (fused append + decode on every
    layer) captured once and replayed after each later prepare_decode_step:
    the kernels read each step's plan, lengths and page ids from the cache's
    step buffer, so every replay equals an eager twin cache bit for bit
    (outputs and cache contents), across page allocations, while
    decode_graph_key() holds; when it changes (here a request outgrows the
    small-batch schedule) the step is captured again."""
    from gpu_offloading_amd.kv_cache import PagedKVCache

    layers, hkv, hq = 3, 8, 32
    seqs, lens = [0, 1, 2], [100, 46, 250]

    def make():
        c = PagedKVCache(layers, hkv, 128, max_seqs=4, max_seq_len=512, num_qo_heads=hq,
                         kv_page_budget=96, device=gpu, workspace_bytes=1 << 22,
                         staging_bytes=1 << 20)
        c.fill_kv_random(1.0, generator=torch.Generator(device=gpu).manual_seed(7))
        for s, ln in zip(seqs, lens):
            c.ensure_pages(s, (ln + 15) // 16)
        c.advance(seqs, lens)
        return c

    eager, graphed = make(), make()
    g = torch.Generator(device=gpu).manual_seed(8)
    bf = torch.bfloat16
    q = [torch.zeros(3, hq, 128, dtype=bf, device=gpu) for _ in range(layers)]
    k = [torch.zeros(3, hkv, 128, dtype=bf, device=gpu) for _ in range(layers)]
    v = [torch.zeros(3, hkv, 128, dtype=bf, device=gpu) for _ in range(layers)]
    out_e = [torch.empty_like(t) for t in q]
    out_g = [torch.empty_like(t) for t in q]
    graph, key, captures, reuses, kinds = None, None, 0, 0, set()
    for step in range(12):
        for t in q + k + v:   # eager work between replays: new inputs in place
            t.copy_(torch.randn(t.shape, generator=g, device=gpu).to(bf))
        for c in (eager, graphed):
            for s in seqs:
                c.ensure_pages(s, (int(c._seq_lens_cpu[s]) + 1 + 15) // 16)
            c.prepare_decode_step(seqs)
        for layer in range(layers):
            eager.append_and_decode(layer, k[layer], v[layer], q[layer], out=out_e[layer])
        kinds.add(graphed._decode_wrapper.schedule.small_batch)
        if graphed.decode_graph_key() != key:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for layer in range(layers):
                    graphed.append_and_decode(layer, k[layer], v[layer], q[layer],
                                              out=out_g[layer])
            key = graphed.decode_graph_key()
            captures += 1
        else:
            reuses += 1
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(layers):
            assert torch.equal(out_g[layer], out_e[layer]), (step, layer)
            assert torch.equal(graphed.k_cache[layer], eager.k_cache[layer]), (step, layer)
            assert torch.equal(graphed.v_cache[layer], eager.v_cache[layer]), (step, layer)
    # Both schedules ran: small-batch for steps 0-5, then request 2 passed 16
    # pages (257 tokens) at step 6.  Each was captured once and replayed for
    # the other steps, the first across request 1's new page at step 2 (49
    # tokens).
    assert kinds == {0, 1}
    assert captures == 2 and reuses == 10
    assert [int(x) for x in graphed._seq_lens_cpu[:3]] == [112, 58, 262]
    assert graphed.seq_pages(1) == 4


def test_decode_graph_key_is_empty_when_the_step_buffer_plan_is_not_current(gpu):
    """decode_graph_key() names the decode step's buffer only while its plan
    is the one the wrapper runs: after a mixed step (whose plan lives in that
    step's own upload) it is empty, so no graph captured for a decode step is
    replayed against another plan; the next decode step restores it."""
    from gpu_offloading_amd.kv_cache import PagedKVCache

    c = PagedKVCache(1, 8, 128, max_seqs=4, max_seq_len=512, num_qo_heads=32,
                     kv_page_budget=64, device=gpu, workspace_bytes=1 << 22,
                     staging_bytes=1 << 20)
    assert c.decode_graph_key() == ()
    c.ensure_pages(0, 3)
    c.ensure_pages(1, 2)
    c.advance([0, 1], [40, 20])
    for s, ln in ((0, 41), (1, 21)):
        c.ensure_pages(s, (ln + 15) // 16)
    c.prepare_decode_step([0, 1])
    key = c.decode_graph_key()
    assert key != ()
    c.ensure_pages(0, 3)
    c.ensure_pages(2, 2)
    c.prepare_step(decode_seq_ids=[0], prefill_seq_ids=[2], prefill_lens=[17])
    assert c.decode_graph_key() == ()
    for s in (0, 1):
        c.ensure_pages(s, (int(c._seq_lens_cpu[s]) + 1 + 15) // 16)
    c.prepare_decode_step([0, 1])
    assert c.decode_graph_key() == key
