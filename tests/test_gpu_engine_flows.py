"""Engine-level flows of the reference's own GPU tests, restated over
PagedKVCache:

* static vs dynamic pages (src/MoE/tests/test_dynamic_pages.py:275-378): the
  same decode steps over identity block tables and over pages taken from a
  shuffled pool give the same attention (here bit for bit: the schedule
  depends on page counts, not ids), and every page is free at the end;
* N-chunk vs single-shot prefill (test_chunked_prefill_comprehensive.py:
  106-147, 301-335): a prompt prefilled as continuation chunks attends like
  the one-shot prefill of the whole prompt (bit for bit: each query row walks
  the same 64-key tiles from key 0)."""
import numpy as np
import pytest
import torch

from gpu_offloading_amd import workloads
from helpers import u16
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu


def test_static_and_dynamic_pages_decode_alike(gpu):
    from gpu_offloading_amd.kv_cache import PagedKVCache

    steps, hkv, hq, max_len = 1000, 8, 32, 1200
    kw = dict(num_qo_heads=hq, device=gpu, workspace_bytes=1 << 22, staging_bytes=1 << 20)
    static = PagedKVCache(1, hkv, 128, max_seqs=2, max_seq_len=max_len, **kw)
    dyn = PagedKVCache(1, hkv, 128, max_seqs=2, max_seq_len=max_len, kv_page_budget=160,
                       free_page_order=workloads.randperm(160, 42), **kw)
    g = torch.Generator(device=gpu).manual_seed(42)
    prompt = [37, 150]
    n = sum(prompt)
    k = torch.randn(n, hkv, 128, generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn(n, hkv, 128, generator=g, device=gpu).to(torch.bfloat16)
    for c in (static, dyn):
        if c is dyn:
            for s, ln in enumerate(prompt):
                c.ensure_pages(s, (ln + 15) // 16)
        c.append(0, k, v, c.slot_mapping([0, 1], prompt))
        c.advance([0, 1], prompt)
    for step in range(steps):
        kn = torch.randn(2, hkv, 128, generator=g, device=gpu).to(torch.bfloat16)
        vn = torch.randn(2, hkv, 128, generator=g, device=gpu).to(torch.bfloat16)
        q = torch.randn(2, hq, 128, generator=g, device=gpu).to(torch.bfloat16)
        for s in (0, 1):
            dyn.ensure_pages(s, (int(dyn._seq_lens_cpu[s]) + 1 + 15) // 16)
        outs = []
        for c in (static, dyn):
            c.prepare_decode_step([0, 1])
            outs.append(c.append_and_decode(0, kn, vn, q))
        if step % 100 == 99:
            torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), step
    assert [int(x) for x in dyn._seq_lens_cpu] == [37 + steps, 150 + steps]
    assert dyn.pages_in_use == (37 + steps + 15) // 16 + (150 + steps + 15) // 16
    for s in (0, 1):
        dyn.free_seq(s)
    assert dyn.pages_in_use == 0 and dyn.pages_free == 160
    assert (dyn.block_table == -1).all()


@pytest.mark.parametrize("chunks", [[520], [200, 256, 64], [1, 128, 391]])
def test_chunked_prefill_equals_single_shot(gpu, chunks):
    from gpu_offloading_amd.kv_cache import PagedKVCache

    total, hkv, hq = sum(chunks), 8, 32
    g = torch.Generator(device=gpu).manual_seed(43)
    k = torch.randn(total, hkv, 128, generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn(total, hkv, 128, generator=g, device=gpu).to(torch.bfloat16)
    q = torch.randn(total, hq, 128, generator=g, device=gpu).to(torch.bfloat16)
    outs = []
    for plan in ([total], chunks):
        c = PagedKVCache(1, hkv, 128, max_seqs=1, max_seq_len=total + 16, num_qo_heads=hq,
                         kv_page_budget=64, free_page_order=workloads.randperm(64, 44),
                         device=gpu, workspace_bytes=1 << 20, staging_bytes=1 << 20)
        pieces, at = [], 0
        for n in plan:
            c.ensure_pages(0, (at + n + 15) // 16)
            slots = c.prepare_prefill_chunk([0], [n])
            c.append(0, k[at:at + n], v[at:at + n], slots)
            pieces.append(c.prefill(0, q[at:at + n]))
            at += n
        outs.append(torch.cat(pieces))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    # and the one-shot result is causal attention over the prompt (oracle)
    kc = np.zeros((64, 16, hkv, 128), np.uint16)
    vc = np.zeros_like(kc)
    pages = workloads.randperm(64, 44)[:(total + 15) // 16]
    pos = np.arange(total)
    slots = np.asarray(pages, np.int64)[pos // 16] * 16 + pos % 16
    orc.reshape_and_cache(u16(k), u16(v), kc, vc, slots)
    kvi, lpl = orc.plan_decode([total])
    idx = np.asarray(pages, np.int32)
    ref, _ = orc.paged_prefill(u16(q), kc, vc, np.array([0, total], np.int32), kvi, idx, lpl)
    err = np.abs(outs[0].float().cpu().numpy() - ref)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3
