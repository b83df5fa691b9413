"""A randomized continuous-batching run of PagedKVCache on the GPU against a
CPU model that keeps every sequence's K/V rows in order: admissions with a
prompt append, decode steps through the one-copy step setup and the fused
append + decode, swap-outs to pinned memory, swap-ins into any free slot,
and finished sequences freed -- on a tight, shuffled page pool.  Each step's
attention must match fp32 attention over the model's rows (max 2e-2 / mean
2e-3), the block table must stay a bijection onto the pages in use, and the
pool must be whole at the end."""
import numpy as np
import pytest
import torch

from gpu_offloading_amd import workloads
from helpers import assert_attn_close, u16
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu

HKV, HQ, D, SLOTS, BUDGET = 8, 32, 128, 6, 120


def _attend(q, k, v):
    """fp32 attention of q [Hq, D] over rows k, v [n, Hkv, D] (bf16 bits)."""
    qf, kf, vf = (orc.bf16_to_f32(x) for x in (q, k, v))
    g = HQ // HKV
    out = np.empty((HQ, D), np.float32)
    for hq in range(HQ):
        s = kf[:, hq // g] @ qf[hq] / np.sqrt(D)
        p = np.exp(s - s.max())
        out[hq] = (p / p.sum()) @ vf[:, hq // g]
    return out


def test_random_batching_with_swaps_matches_the_model(gpu):
    from gpu_offloading_amd.kv_cache import PagedKVCache

    rng = np.random.default_rng(2024)
    g = torch.Generator(device=gpu).manual_seed(2025)
    cache = PagedKVCache(1, HKV, D, max_seqs=SLOTS, max_seq_len=1024, num_qo_heads=HQ,
                         kv_page_budget=BUDGET, free_page_order=workloads.randperm(BUDGET, 7),
                         device=gpu, workspace_bytes=1 << 24, staging_bytes=3 * 2 * 65536)
    rows = {}        # slot -> (K rows, V rows) as uint16 [n, Hkv, D]
    swapped = []     # (handle, K rows, V rows)
    tally = dict(finish=0, swap_out=0, swap_in=0, admit=0, fused=0)

    def rand_rows(n):
        k = torch.randn(n, HKV, D, generator=g, device=gpu).to(torch.bfloat16)
        v = torch.randn(n, HKV, D, generator=g, device=gpu).to(torch.bfloat16)
        return k, v

    def free_slots():
        return [s for s in range(SLOTS) if s not in rows]

    for step in range(300):
        u = rng.random()
        if u < 0.12 and rows:                                   # finish a sequence
            s = int(rng.choice(list(rows)))
            cache.free_seq(s)
            del rows[s]
            tally["finish"] += 1
        elif u < 0.24 and len(rows) > 1:                        # preempt by swap
            s = int(rng.choice(list(rows)))
            h = cache.swap_out([s])
            swapped.append((h,) + rows.pop(s))
            tally["swap_out"] += 1
        elif u < 0.36 and swapped and free_slots():             # resume elsewhere
            h, k, v = swapped[0]
            need = (len(k) + 1 + 15) // 16
            cache.synchronize_swaps()
            if cache.pages_free >= need + 2:
                s = int(rng.choice(free_slots()))
                cache.swap_in(h, seq_ids=[s])
                rows[s] = (k, v)
                swapped.pop(0)
                tally["swap_in"] += 1
        if len(rows) < 3 and free_slots():                      # admit with a prompt
            n = int(rng.integers(1, 300))
            cache.synchronize_swaps()
            if cache.pages_free >= (n + 1 + 15) // 16 + 4:
                s = int(rng.choice(free_slots()))
                cache.ensure_pages(s, (n + 15) // 16)
                k, v = rand_rows(n)
                slots = cache.slot_mapping([s], [n])
                cache.append(0, k, v, slots)
                cache.advance([s], [n])
                rows[s] = (u16(k), u16(v))
                tally["admit"] += 1
        if not rows:
            continue
        # preempt (swap out the longest) while the step's new pages do not fit
        while True:
            cache.synchronize_swaps()
            need = sum(max(0, (len(rows[x][0]) + 1 + 15) // 16 - cache.seq_pages(x)) for x in rows)
            if need <= cache.pages_free or len(rows) == 1:
                break
            s = max(rows, key=lambda x: len(rows[x][0]))
            h = cache.swap_out([s])
            swapped.append((h,) + rows.pop(s))
            tally["swap_out"] += 1
        seqs = list(rows)
        rng.shuffle(seqs)
        for s in seqs:
            cache.ensure_pages(s, (len(rows[s][0]) + 1 + 15) // 16)
        cache.prepare_decode_step(seqs)
        tally["fused"] += int(cache._decode_wrapper.fused_append_supported)
        k, v = rand_rows(len(seqs))
        q = torch.randn(len(seqs), HQ, D, generator=g, device=gpu).to(torch.bfloat16)
        out = cache.append_and_decode(0, k, v, q)
        ku, vu, qu = u16(k), u16(v), u16(q)
        for i, s in enumerate(seqs):
            rows[s] = (np.concatenate([rows[s][0], ku[i:i + 1]]),
                       np.concatenate([rows[s][1], vu[i:i + 1]]))
        got = out.float().cpu().numpy()
        ref = np.stack([_attend(qu[i], *rows[s]) for i, s in enumerate(seqs)])
        assert_attn_close(got, ref)
        # the table maps every resident token's page to a distinct page
        bt = cache.block_table.cpu().numpy()
        used = np.concatenate([bt[s, :(len(rows[s][0]) + 15) // 16] for s in rows])
        assert (used >= 0).all() and len(np.unique(used)) == len(used), step
        assert [int(cache._seq_lens_cpu[s]) for s in rows] == [len(rows[s][0]) for s in rows]
    # bring everything back, check the bytes, then free it all
    cache.synchronize_swaps()
    for h, k, v in swapped:
        cache.synchronize_swaps()
        if not free_slots() or cache.pages_free < (len(k) + 15) // 16:
            break
        s = free_slots()[0]
        cache.swap_in(h, seq_ids=[s], wait=True)
        rows[s] = (k, v)
    torch.cuda.synchronize()
    bt = cache.block_table.cpu().numpy()
    for s, (k, v) in rows.items():
        pages = bt[s, :(len(k) + 15) // 16]
        kk = u16(cache.k_cache[0][torch.from_numpy(pages).long().to(gpu)]).reshape(-1, HKV, D)
        vv = u16(cache.v_cache[0][torch.from_numpy(pages).long().to(gpu)]).reshape(-1, HKV, D)
        assert np.array_equal(kk[:len(k)], k) and np.array_equal(vv[:len(v)], v)
    for s in list(rows):
        cache.free_seq(s)
    cache.synchronize_swaps()
    assert cache.pages_in_use == 0 and cache.pages_free == BUDGET
    assert min(tally.values()) >= 5, tally
