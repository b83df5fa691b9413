"""Parity of the exact path bench.py times: the configuration-2 decode step
(Mixtral shape, 32 layers, 64 sequences with context U[512, 4096], the seeded
permuted pool), built the way the bench builds it, stepped the way the bench
steps it (ensure_pages, prepare_decode_step, then one fused append_and_decode
launch per layer).

* One layer at the bench shape: the fused launch equals the two-call path
  (reshape_and_cache_flash, then run) bit for bit -- cache bytes, output and
  lse -- and the oracle within max 2e-2 / mean 2e-3.
* The 32-layer loop after several steps: layers 0 and 31 hold exactly the
  oracle's cache (the initial bytes plus every step's rows at the oracle's
  slots), and their last-step outputs match the oracle's attention.
"""
import numpy as np
import pytest
import torch

from gpu_offloading_amd import workloads
from gpu_offloading_amd.kv_cache import PagedKVCache
from helpers import assert_attn_close, u16
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu


def _bench_cache(gpu, num_layers, seed=0):
    """The bench's configuration-2 cache (bench.py build_cfg2_cache)."""
    cfg = workloads.config2(seed=seed)
    sh = cfg.shape
    seqs = list(range(len(cfg.seq_lens)))
    cache = PagedKVCache(num_layers, sh.num_kv_heads, sh.head_dim, max_seqs=len(seqs),
                         max_seq_len=max(cfg.seq_lens) + cfg.extra["extra_steps"] + 16,
                         num_qo_heads=sh.num_qo_heads, kv_page_budget=cfg.total_pages,
                         free_page_order=cfg.free_order, device=gpu)
    for s, ln in zip(seqs, cfg.seq_lens):
        cache.ensure_pages(s, (ln + 15) // 16)
    cache.advance(seqs, cfg.seq_lens)
    g = torch.Generator(device=gpu).manual_seed(seed + 100)
    for kc, vc in zip(cache.k_cache, cache.v_cache):
        kc.normal_(0.0, 1.0, generator=g)
        vc.normal_(0.0, 1.0, generator=g)
    return cfg, cache, seqs


def _rows(gpu, shape, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    return torch.randn(*shape, device=gpu, generator=g).to(torch.bfloat16)


def _oracle_decode(cache, layer, seqs, q):
    lens = [int(cache._seq_lens_cpu[s]) for s in seqs]
    indptr, lpl = orc.plan_decode(lens)
    idx = orc.page_indices(cache.block_table.cpu().numpy(), seqs, indptr)
    return orc.paged_decode(u16(q), u16(cache.k_cache[layer]), u16(cache.v_cache[layer]),
                            indptr, idx, lpl)


def test_fused_step_equals_two_calls_at_the_bench_shape(gpu):
    print("bench path: cfg2 one layer, fused vs two calls", flush=True)
    cfg, a, seqs = _bench_cache(gpu, 1)
    _, b, _ = _bench_cache(gpu, 1)
    sh = cfg.shape
    B = len(seqs)
    k = _rows(gpu, (B, sh.num_kv_heads, sh.head_dim), 1)
    v = _rows(gpu, (B, sh.num_kv_heads, sh.head_dim), 2)
    q = _rows(gpu, (B, sh.num_qo_heads, sh.head_dim), 3)
    for c in (a, b):
        for s in seqs:
            c.ensure_pages(s, (int(c._seq_lens_cpu[s]) + 1 + 15) // 16)
    slots = a.prepare_decode_step(seqs)
    a.append(0, k, v, slots)
    out_a, lse_a = a.decode(0, q, return_lse=True)
    b.prepare_decode_step(seqs)
    assert b._decode_wrapper.fused_append_supported     # the bench's launch
    sched = b._decode_wrapper.schedule
    assert sched.max_partitions > 1                      # split requests and the merge
    out_b, lse_b = b.append_and_decode(0, k, v, q, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(a.kv_cache[0], b.kv_cache[0])
    assert torch.equal(out_a, out_b) and torch.equal(lse_a, lse_b)
    ref, ref_lse = _oracle_decode(b, 0, seqs, q)
    assert_attn_close(out_b.float().cpu().numpy(), ref)
    assert np.abs(lse_b.cpu().numpy() - ref_lse).max() < 2e-3


def test_bench_step_loop_matches_the_oracle_after_several_steps(gpu):
    steps, check = 4, (0, 31)
    print(f"bench path: cfg2 32-layer loop, {steps} steps, layers {check}", flush=True)
    cfg, cache, seqs = _bench_cache(gpu, 32)
    sh = cfg.shape
    B, L = len(seqs), sh.num_layers
    init = {l: (u16(cache.k_cache[l]), u16(cache.v_cache[l])) for l in check}
    appended = {l: ([], []) for l in check}
    all_slots = []
    outs = {}
    for step in range(steps):
        for s in seqs:
            cache.ensure_pages(s, (int(cache._seq_lens_cpu[s]) + 1 + 15) // 16)
        slots = cache.prepare_decode_step(seqs)
        assert cache._decode_wrapper.fused_append_supported
        all_slots.append(slots.cpu().numpy())
        for layer in range(L):
            base = 1000 * step + 3 * layer
            k = _rows(gpu, (B, sh.num_kv_heads, sh.head_dim), base)
            v = _rows(gpu, (B, sh.num_kv_heads, sh.head_dim), base + 1)
            q = _rows(gpu, (B, sh.num_qo_heads, sh.head_dim), base + 2)
            out = cache.append_and_decode(layer, k, v, q)
            if layer in check:
                appended[layer][0].append(u16(k))
                appended[layer][1].append(u16(v))
                outs[layer] = (q, out)
    torch.cuda.synchronize()
    slots_np = np.concatenate(all_slots)
    for layer in check:
        ek, ev = init[layer]
        orc.reshape_and_cache(np.concatenate(appended[layer][0]),
                              np.concatenate(appended[layer][1]), ek, ev, slots_np)
        assert np.array_equal(u16(cache.k_cache[layer]), ek), f"layer {layer}: K cache"
        assert np.array_equal(u16(cache.v_cache[layer]), ev), f"layer {layer}: V cache"
        q, out = outs[layer]
        ref, _ = _oracle_decode(cache, layer, seqs, q)
        assert_attn_close(out.float().cpu().numpy(), ref)
