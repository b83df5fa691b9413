"""GPU parity of the one-upload mixed step (PagedKVCache.prepare_step): the
engine's step() with decode requests, new prompts and continuation chunks in
one batch (src/MoE/moe_engine.py:2555-2742, setup :3475-3556, continuation
plan :3649-3728).  Checked against the oracle on a CPU model of every
sequence's rows:

* the slot mapping equals orc.step_slot_mapping on the oracle's page pool
  ([decode | new prefill | continuation], positions from the lengths before
  the step, -1 padding to graph_n), bit for bit;
* lengths after the step: decode + 1, prompt length, offset + chunk;
* the appended rows land where the model says (gather is bit-exact);
* decode attention matches orc.paged_decode and continuation attention
  matches orc.paged_prefill (causal, aligned to the end of the cache), both
  within max 2e-2 / mean 2e-3, over the model's rows.
Two steps in a row: the second decodes the first step's new prompts."""
import numpy as np
import pytest
import torch

from gpu_offloading_amd import workloads
from gpu_offloading_amd.kv_cache import PagedKVCache
from helpers import assert_attn_close, oracle_decode_rows, randn_bf16, u16
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu

HKV, HQ, D = 8, 32, 128


def _paged_from_rows(k_rows, v_rows):
    """Consecutive pages holding each request's rows (for orc.paged_prefill)."""
    lens = [len(k) for k in k_rows]
    indptr, lpl = orc.plan_decode(lens)
    kc = np.zeros((max(int(indptr[-1]), 1), 16, HKV, D), np.uint16)
    vc = np.zeros_like(kc)
    for b, (k, v) in enumerate(zip(k_rows, v_rows)):
        kc[indptr[b]:indptr[b + 1]].reshape(-1, HKV, D)[:len(k)] = k
        vc[indptr[b]:indptr[b + 1]].reshape(-1, HKV, D)[:len(v)] = v
    return kc, vc, indptr, np.arange(int(indptr[-1]), dtype=np.int32), lpl


def test_mixed_steps_match_the_oracle(gpu):
    layers, ms, total = 2, 8, 220
    order = workloads.randperm(total, 80)
    cache = PagedKVCache(layers, HKV, D, max_seqs=ms, max_seq_len=512, num_qo_heads=HQ,
                         kv_page_budget=total, free_page_order=order, device=gpu,
                         workspace_bytes=1 << 24, staging_bytes=1 << 20)
    pool = orc.FifoPagePool(total, ms, cache.max_pages_per_seq, free_order=order)
    rows = {(s, l): [np.zeros((0, HKV, D), np.uint16)] * 2 for s in range(ms)
            for l in range(layers)}
    lens = np.zeros(ms, np.int64)

    # History: sequences 0-2 decoding, 3-4 mid-prompt (one chunk done).
    hist = {0: 50, 1: 17, 2: 130, 3: 40, 4: 64}
    for s, n in hist.items():
        cache.ensure_pages(s, (n + 15) // 16)
        pool.ensure_pages(s, (n + 15) // 16)
    slots = cache.slot_mapping(list(hist), list(hist.values()))
    ntok = sum(hist.values())
    for layer in range(layers):
        k = randn_bf16((ntok, HKV, D), 100 + layer, device=gpu)
        v = randn_bf16((ntok, HKV, D), 110 + layer, device=gpu)
        cache.append(layer, k, v, slots)
        off = 0
        for s, n in hist.items():
            rows[s, layer] = [u16(k[off:off + n]), u16(v[off:off + n])]
            off += n
    cache.advance(list(hist), list(hist.values()))
    for s, n in hist.items():
        lens[s] = n

    steps = [
        dict(decode=[2, 0, 1], prefill=[6, 5], plen=[100, 37], cont=[4, 3], clen=[30, 70]),
        dict(decode=[5, 0, 2, 6, 1], prefill=[7], plen=[16], cont=[3], clen=[48]),
    ]
    for si, st in enumerate(steps):
        print(f"mixed step {si}: {st}", flush=True)
        dec, pre, plen, con, clen = st["decode"], st["prefill"], st["plen"], st["cont"], st["clen"]
        counts = [1] * len(dec) + plen + clen
        seqs = dec + pre + con
        for s, c in zip(seqs, counts):
            cache.ensure_pages(s, (int(lens[s]) + c + 15) // 16)
            pool.ensure_pages(s, (int(lens[s]) + c + 15) // 16)
        graph_n = sum(counts) + 5
        slots = cache.prepare_step(dec, pre, plen, con, clen, graph_n=graph_n)
        want, _ = orc.step_slot_mapping(pool.block_table, seqs, counts, lens, graph_n)
        assert np.array_equal(slots.cpu().numpy(), want)
        before = lens.copy()
        for s, c in zip(seqs, counts):
            lens[s] += c
        assert np.array_equal(cache.seq_lens.cpu().numpy(), lens)
        assert np.array_equal(cache._seq_lens_cpu.numpy(), lens)
        assert np.array_equal(cache.block_table.cpu().numpy(), pool.block_table)

        n_tok = sum(counts)
        starts = np.concatenate([[0], np.cumsum(counts)])
        for layer in range(layers):
            k = randn_bf16((n_tok, HKV, D), 1000 * si + 10 * layer + 1, device=gpu)
            v = randn_bf16((n_tok, HKV, D), 1000 * si + 10 * layer + 2, device=gpu)
            cache.append(layer, k, v, slots[:n_tok])
            for i, s in enumerate(seqs):
                a, b = starts[i], starts[i + 1]
                rows[s, layer] = [np.concatenate([rows[s, layer][0], u16(k[a:b])]),
                                  np.concatenate([rows[s, layer][1], u16(v[a:b])])]
            # decode requests
            qd = randn_bf16((len(dec), HQ, D), 1000 * si + 10 * layer + 3, device=gpu)
            out = cache.decode(layer, qd)
            ref, _ = oracle_decode_rows(u16(qd), [rows[s, layer][0] for s in dec],
                                        [rows[s, layer][1] for s in dec])
            assert_attn_close(out.float().cpu().numpy(), ref)
            # continuation chunks: their query rows, chunk after chunk
            qc = randn_bf16((sum(clen), HQ, D), 1000 * si + 10 * layer + 4, device=gpu)
            outc = cache.prefill(layer, qc)
            kc, vc, kvi, idx, lpl = _paged_from_rows([rows[s, layer][0] for s in con],
                                                     [rows[s, layer][1] for s in con])
            qo = np.concatenate([[0], np.cumsum(clen)]).astype(np.int32)
            refc, _ = orc.paged_prefill(u16(qc), kc, vc, qo, kvi, idx, lpl, causal=True)
            assert_attn_close(outc.float().cpu().numpy(), refc)
            # the cache holds every sequence's rows exactly
            gk, gv = cache.gather(layer, seqs)
            torch.cuda.synchronize()
            assert np.array_equal(u16(gk), np.concatenate([rows[s, layer][0] for s in seqs]))
            assert np.array_equal(u16(gv), np.concatenate([rows[s, layer][1] for s in seqs]))
        assert (before[pre] == 0).all()


def test_mixed_step_refuses_bad_requests(gpu):
    cache = PagedKVCache(1, HKV, D, max_seqs=4, max_seq_len=256, num_qo_heads=HQ,
                         kv_page_budget=64, device=gpu, workspace_bytes=1 << 22,
                         staging_bytes=1 << 20)
    cache.ensure_pages(0, 2)
    cache.advance([0], [20])
    with pytest.raises(ValueError, match="distinct"):
        cache.prepare_step([0], [0], [5])                  # one sequence twice
    with pytest.raises(RuntimeError, match="must be empty"):
        cache.ensure_pages(1, 1)
        cache.advance([1], [3])
        cache.prepare_step([], [1], [4])                   # a prompt into a used slot
    with pytest.raises(RuntimeError, match="no page"):
        cache.prepare_step([], [2], [40])                  # no pages allocated
    with pytest.raises(ValueError, match="graph_n"):
        cache.prepare_step([0], graph_n=0)
    with pytest.raises(ValueError, match="positive"):
        cache.prepare_step([], [], [], [0], [0])
    # the cache is untouched by the refused calls
    assert cache._seq_lens_cpu[0] == 20 and cache._seq_lens_cpu[2] == 0
