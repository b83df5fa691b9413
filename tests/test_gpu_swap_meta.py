"""GPU parity of block eviction/restore (bit-exact round trips) and of the
step-setup metadata kernels (slot mapping, page-index flattening)."""
import numpy as np
import pytest
import torch

from gpu_offloading_amd import ops, workloads
from helpers import randn_bf16, u16
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu


def _caches(layers, blocks, h, d, seed, gpu):
    ks = [randn_bf16((blocks, 16, h, d), seed + 2 * i, device=gpu) for i in range(layers)]
    vs = [randn_bf16((blocks, 16, h, d), seed + 2 * i + 1, device=gpu) for i in range(layers)]
    return ks, vs


def test_gather_scatter_blocks_vs_oracle(gpu):
    ks, vs = _caches(1, 64, 16, 128, 1, gpu)
    ids = np.array(workloads.randperm(64, 2)[:17], np.int32)
    staging = torch.empty(17 * 2 * ops.block_bytes(ks[0]), dtype=torch.uint8, device=gpu)
    ops.gather_blocks(ks[0], vs[0], torch.from_numpy(ids).to(gpu), staging)
    ref = orc.gather_blocks(u16(ks[0]), u16(vs[0]), ids)
    assert np.array_equal(staging.cpu().numpy().reshape(ref.shape), ref)
    # scatter the staged image into other blocks
    dst = np.array(workloads.randperm(64, 3)[:17], np.int32)
    k2, v2 = _caches(1, 64, 16, 128, 50, gpu)
    ek, ev = u16(k2[0]), u16(v2[0])
    ops.scatter_blocks(staging, torch.from_numpy(dst).to(gpu), k2[0], v2[0])
    orc.scatter_blocks(ref, dst, ek, ev)
    assert np.array_equal(u16(k2[0]), ek) and np.array_equal(u16(v2[0]), ev)


@pytest.mark.parametrize("staging_blocks", [1, 5, 1000])
def test_swap_out_in_round_trip_bit_exact(gpu, staging_blocks):
    layers, blocks, h, d = 3, 96, 16, 128
    ks, vs = _caches(layers, blocks, h, d, 10, gpu)
    snap = ([k.clone() for k in ks], [v.clone() for v in vs])
    ids = torch.tensor(workloads.randperm(blocks, 4)[:24], dtype=torch.int32, device=gpu)
    bb = ops.block_bytes(ks[0])
    host = torch.empty(layers * 24 * 2 * bb, dtype=torch.uint8, pin_memory=True)
    staging = torch.empty(staging_blocks * 2 * bb, dtype=torch.uint8, device=gpu)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    ops.swap_out_blocks(ks, vs, ids, host, staging, stream=side)
    side.synchronize()
    # the host image is the oracle's staging image, layer by layer
    ref = np.concatenate([orc.gather_blocks(u16(k), u16(v), ids.cpu().numpy()).ravel()
                          for k, v in zip(ks, vs)])
    assert np.array_equal(host.numpy(), ref)
    # clobber the evicted blocks, then restore into the same ids
    for k, v in zip(ks, vs):
        k[ids.long()] = 0
        v[ids.long()] = 0
    torch.cuda.synchronize()
    ops.swap_in_blocks(host, ids, ks, vs, staging, stream=side)
    side.synchronize()
    for a, b in zip(ks + vs, snap[0] + snap[1]):
        assert torch.equal(a, b)


def test_swap_in_to_different_blocks(gpu):
    layers, blocks = 2, 64
    ks, vs = _caches(layers, blocks, 8, 128, 30, gpu)
    perm = workloads.randperm(blocks, 5)
    src = torch.tensor(perm[:10], dtype=torch.int32, device=gpu)
    dst = torch.tensor(perm[10:20], dtype=torch.int32, device=gpu)
    bb = ops.block_bytes(ks[0])
    host = torch.empty(layers * 10 * 2 * bb, dtype=torch.uint8, pin_memory=True)
    staging = torch.empty(4 * 2 * bb, dtype=torch.uint8, device=gpu)
    before = [(k.clone(), v.clone()) for k, v in zip(ks, vs)]
    ops.swap_out_blocks(ks, vs, src, host, staging)
    ops.swap_in_blocks(host, dst, ks, vs, staging)
    torch.cuda.synchronize()
    untouched = torch.ones(blocks, dtype=torch.bool)
    untouched[dst.long().cpu()] = False
    for (k0, v0), k, v in zip(before, ks, vs):
        assert torch.equal(k[dst.long()], k0[src.long()])
        assert torch.equal(v[dst.long()], v0[src.long()])
        assert torch.equal(k[untouched.to(gpu)], k0[untouched.to(gpu)])


def test_swap_rejects_pageable_host_buffer(gpu):
    ks, vs = _caches(1, 8, 8, 128, 40, gpu)
    ids = torch.tensor([1, 2], dtype=torch.int32, device=gpu)
    staging = torch.empty(2 * 2 * ops.block_bytes(ks[0]), dtype=torch.uint8, device=gpu)
    with pytest.raises(RuntimeError):
        ops.swap_out_blocks(ks, vs, ids, torch.empty(staging.numel(), dtype=torch.uint8), staging)


def test_compute_slot_mapping_vs_oracle(gpu):
    rng = np.random.default_rng(0)
    max_seqs, width = 12, 40
    pool = orc.FifoPagePool(400, max_seqs, width, free_order=workloads.randperm(400, 9))
    computed = rng.integers(0, 300, max_seqs).astype(np.int32)
    seq_ids = [3, 7, 0, 11, 5]
    new = [1, 1, 37, 100, 16]  # two decode tokens, then prefill/continuation chunks
    for s, n in zip(seq_ids, new):
        pool.ensure_pages(s, (int(computed[s]) + n + 15) // 16)
    graph_n = sum(new) + 9
    ref_slots, ref_pos = orc.step_slot_mapping(pool.block_table, seq_ids, new, computed, graph_n)
    qsl = np.zeros(len(new) + 1, np.int32)
    np.cumsum(new, out=qsl[1:])
    slots = torch.empty(graph_n, dtype=torch.int64, device=gpu)
    pos = torch.empty(graph_n, dtype=torch.int32, device=gpu)
    ops.compute_slot_mapping(torch.from_numpy(pool.block_table).to(gpu),
                             torch.tensor(seq_ids, dtype=torch.int32, device=gpu),
                             torch.from_numpy(qsl).to(gpu), torch.from_numpy(computed).to(gpu),
                             sum(new), slots, pos)
    assert np.array_equal(slots.cpu().numpy(), ref_slots)
    assert np.array_equal(pos.cpu().numpy(), ref_pos)


def test_copy_page_indices_vs_oracle(gpu):
    max_seqs, width = 10, 300
    pool = orc.FifoPagePool(2000, max_seqs, width, free_order=workloads.randperm(2000, 11))
    lens = [5, 1000, 16, 4096, 1, 33]
    seq_ids = [9, 2, 4, 0, 7, 3]
    for s, ln in zip(seq_ids, lens):
        pool.ensure_pages(s, (ln + 15) // 16)
    indptr, _ = orc.plan_decode(lens)
    ref = orc.page_indices(pool.block_table, seq_ids, indptr)
    out = torch.full((int(indptr[-1]) + 5,), -7, dtype=torch.int32, device=gpu)
    ops.copy_page_indices(torch.from_numpy(pool.block_table).to(gpu), torch.from_numpy(indptr).to(gpu),
                          out, seq_ids=torch.tensor(seq_ids, dtype=torch.int32, device=gpu))
    got = out.cpu().numpy()
    assert np.array_equal(got[:-5], ref) and (got[-5:] == -7).all()


@pytest.mark.parametrize("staging_blocks", [1, 3, 7, 1000])
def test_cache_swap_chunks_across_layers_bit_exact(gpu, staging_blocks):
    """PagedKVCache.swap_out / swap_in with staging halves of 1, 3, 7 and
    1000 blocks: chunks pack consecutive (layer, block) items of the host
    image across layer boundaries.  The host image equals the oracle's
    layer-by-layer block image, and the restore into other slots is exact."""
    from gpu_offloading_amd.kv_cache import PagedKVCache

    layers, hkv = 3, 2
    per = 2 * 16 * hkv * 128 * 2
    cache = PagedKVCache(layers, hkv, 128, max_seqs=4, max_seq_len=256, kv_page_budget=64,
                         free_page_order=workloads.randperm(64, 80), device=gpu,
                         workspace_bytes=1 << 20, staging_bytes=2 * staging_blocks * per)
    lens = {0: 70, 1: 40, 2: 64}
    for s, ln in lens.items():
        cache.ensure_pages(s, (ln + 15) // 16)
    cache.advance(list(lens), list(lens.values()))
    cache.fill_kv_random(1.0, generator=torch.Generator(device=gpu).manual_seed(81))
    bt = cache.block_table.cpu().numpy()
    pages = {s: bt[s, :(ln + 15) // 16].copy() for s, ln in lens.items()}
    snap = {s: [(cache.k_cache[l][torch.from_numpy(p).long().to(gpu)].clone(),
                 cache.v_cache[l][torch.from_numpy(p).long().to(gpu)].clone())
                for l in range(layers)] for s, p in pages.items()}
    ids = np.concatenate([pages[0], pages[2]])
    ref = np.concatenate([orc.gather_blocks(u16(cache.k_cache[l]), u16(cache.v_cache[l]), ids)
                          .ravel() for l in range(layers)])
    h = cache.swap_out([0, 2])
    cache.synchronize_swaps()
    assert np.array_equal(h.host[:ref.size].numpy(), ref)
    cache.fill_kv_random(1.0, generator=torch.Generator(device=gpu).manual_seed(82))
    keep1 = [(cache.k_cache[l][torch.from_numpy(pages[1]).long().to(gpu)].clone())
             for l in range(layers)]
    cache.swap_in(h, seq_ids=[3, 0], wait=True)
    torch.cuda.synchronize()
    bt = cache.block_table.cpu().numpy()
    for src, dst in ((0, 3), (2, 0)):
        p = torch.from_numpy(bt[dst, :len(pages[src])]).long().to(gpu)
        for l in range(layers):
            assert torch.equal(cache.k_cache[l][p], snap[src][l][0])
            assert torch.equal(cache.v_cache[l][p], snap[src][l][1])
    for l in range(layers):
        assert torch.equal(cache.k_cache[l][torch.from_numpy(pages[1]).long().to(gpu)], keep1[l])
    assert [int(cache._seq_lens_cpu[s]) for s in (3, 0, 1, 2)] == [70, 64, 40, 0]


@pytest.mark.parametrize("staging_blocks", [1, 1000])
def test_reserve_swap_warm_up_leaves_the_caches_untouched(gpu, staging_blocks):
    """reserve_swap's warm-up (copies through the staging, gathers of block 0
    into it) changes no cache byte, runs once, and a swap round trip after
    it is exact; staging of 2 blocks (smaller than the warm-up's 16 MiB
    copies) and of 2000 blocks."""
    from gpu_offloading_amd.kv_cache import PagedKVCache

    layers, hkv = 3, 2
    per = 2 * 16 * hkv * 128 * 2
    cache = PagedKVCache(layers, hkv, 128, max_seqs=2, max_seq_len=256, kv_page_budget=32,
                         free_page_order=workloads.randperm(32, 90), device=gpu,
                         workspace_bytes=1 << 20, staging_bytes=2 * staging_blocks * per)
    cache.ensure_pages(0, 5)
    cache.advance([0], [70])
    cache.fill_kv_random(1.0, generator=torch.Generator(device=gpu).manual_seed(91))
    snap = cache.kv_snapshot()
    cache.reserve_swap()
    cache.reserve_swap()
    torch.cuda.synchronize()
    for l in range(layers):
        assert torch.equal(cache.k_cache[l], snap[0][l])
        assert torch.equal(cache.v_cache[l], snap[1][l])
    pages = cache.block_table.cpu().numpy()[0, :5].copy()
    h = cache.swap_out([0])
    cache.swap_in(h, wait=True)
    torch.cuda.synchronize()
    dst = torch.from_numpy(cache.block_table.cpu().numpy()[0, :5]).long().to(gpu)
    src = torch.from_numpy(pages).long().to(gpu)
    for l in range(layers):
        assert torch.equal(cache.k_cache[l][dst], snap[0][l][src])
        assert torch.equal(cache.v_cache[l][dst], snap[1][l][src])


def test_cfg5_swap_under_decode_round_trip(gpu):
    """Configuration 5's shape (OLMoE MHA 16 x 128, 128 requests x 2048
    tokens on a shuffled 16,384-page pool; 4 of its 16 layers): a seeded
    25% of the requests are swapped out while the other 96 decode, then
    swapped back into other slots; the restored pages are bit-exact and
    the decode of the running requests is unchanged by the swap."""
    from gpu_offloading_amd.kv_cache import PagedKVCache

    cfg = workloads.config5(seed=0)
    L, B = 4, len(cfg.seq_lens)
    cache = PagedKVCache(L, 16, 128, max_seqs=B + 32, max_seq_len=2048 + 64, num_qo_heads=16,
                         kv_page_budget=cfg.total_pages, free_page_order=cfg.free_order,
                         device=gpu, staging_bytes=256 << 20)
    seqs = list(range(B))
    for s in seqs:
        cache.ensure_pages(s, 2048 // 16)
    cache.advance(seqs, cfg.seq_lens)
    cache.fill_kv_random(1.0, generator=torch.Generator(device=gpu).manual_seed(90))
    victims = sorted(workloads.randperm(B, 7)[: B // 4])
    running = [s for s in seqs if s not in set(victims)]
    before = [cache.gather(layer, victims) for layer in range(L)]
    q = torch.randn(len(running), 16, 128, generator=torch.Generator(device=gpu).manual_seed(91),
                    device=gpu).to(torch.bfloat16)
    cache.plan_decode(running)
    ref = [cache.decode(layer, q).clone() for layer in range(L)]
    h = cache.swap_out(victims)
    during = [cache.decode(layer, q) for layer in range(L)]
    cache.synchronize_swaps()
    targets = list(range(B, B + len(victims)))          # resume in other slots
    cache.swap_in(h, seq_ids=targets, wait=True)
    after = [cache.gather(layer, targets) for layer in range(L)]
    torch.cuda.synchronize()
    for layer in range(L):
        assert torch.equal(during[layer], ref[layer])
        for a, b in zip(before[layer], after[layer]):
            assert torch.equal(a, b)
    assert h.bytes_per_direction == L * len(victims) * 128 * 2 * 16 * 16 * 128 * 2


@pytest.mark.parametrize("staging_mib", [8, 64])
def test_c_abi_swap_round_trip_and_rate(gpu, staging_mib):
    """kvc_swap_out / kvc_swap_in through the C entry points: one layer of
    configuration 5's eviction (4096 of 8192 OLMoE blocks, 128 KiB of K+V
    each: 512 MiB each way) through an 8 or 64 MiB staging buffer, restored
    into other block ids bit for bit (the oracle's block image).  The rate is
    printed only: it depends on the box's host link, not on this code."""
    from gpu_offloading_amd import _lib

    print(f"c-abi swap: 512 MiB each way, {staging_mib} MiB staging", flush=True)
    lib = _lib.load()
    nb, n = 8192, 4096
    g = torch.Generator(device=gpu).manual_seed(60)
    kc = torch.empty(nb, 16, 16, 128, dtype=torch.bfloat16, device=gpu).normal_(generator=g)
    vc = torch.empty_like(kc).normal_(generator=g)
    bb = ops.block_bytes(kc)
    src = torch.tensor(workloads.randperm(nb, 61)[:n], dtype=torch.int32, device=gpu)
    dst = torch.tensor(workloads.randperm(nb, 62)[:n], dtype=torch.int32, device=gpu)
    staging = torch.empty(staging_mib << 20, dtype=torch.uint8, device=gpu)
    host = torch.empty(n * 2 * bb, dtype=torch.uint8, pin_memory=True)
    ref = orc.gather_blocks(u16(kc), u16(vc), src.cpu().numpy())
    side = torch.cuda.Stream(device=gpu)
    k2, v2 = torch.zeros_like(kc), torch.zeros_like(vc)
    rates = {}
    for direction in ("out", "in"):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(side)
        if direction == "out":
            st = lib.kvc_swap_out(kc.data_ptr(), vc.data_ptr(), kc.stride(0) * 2, bb, nb,
                                  src.data_ptr(), n, staging.data_ptr(), staging.numel(),
                                  host.data_ptr(), None, side.cuda_stream)
        else:
            st = lib.kvc_swap_in(host.data_ptr(), dst.data_ptr(), n, k2.data_ptr(),
                                 v2.data_ptr(), kc.stride(0) * 2, bb, nb, staging.data_ptr(),
                                 staging.numel(), None, side.cuda_stream)
        assert st == 0, lib.kvc_last_error()
        e1.record(side)
        e1.synchronize()
        rates[direction] = n * 2 * bb / (e0.elapsed_time(e1) * 1e-3) / 1e9
        if direction == "out":
            assert np.array_equal(host.numpy().reshape(ref.shape), ref)
    got = orc.gather_blocks(u16(k2), u16(v2), dst.cpu().numpy())
    assert np.array_equal(got, ref)
    print(f"c-abi swap GB/s ({staging_mib} MiB staging): out {rates['out']:.1f}, "
          f"in {rates['in']:.1f}", flush=True)
