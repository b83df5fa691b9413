"""GPU parity of paged-KV prefill attention (continuation prefill, MFMA)
against the fp32 CPU oracle: max-abs-error <= 2e-2 and mean-abs-error <= 2e-3
on the bf16 output; lse within LSE_TOL.  The kernel sums the row's
probabilities as rounded to bf16 for the P.V product (round to nearest, 8
significant bits: relative error <= 2^-8 per term), so its l is within a
factor 1 +- 2^-8 of the exact sum and lse = m + ln l within ln(1 + 2^-8) =
0.0039 of it, plus fp32 rounding."""
import numpy as np
import pytest
import torch

from gpu_offloading_amd import workloads
from gpu_offloading_amd.decode import BatchDecodeWithPagedKVCacheWrapper
from gpu_offloading_amd.prefill import BatchPrefillWithPagedKVCacheWrapper
from helpers import assert_attn_close, randn_bf16, u16
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu

WS = 16 * 1024 * 1024
LSE_TOL = 4e-3


def _case(q_lens, kv_lens, hq, hkv, seed, d=128, extra_pages=8, device=None):
    need = sum((ln + 15) // 16 for ln in kv_lens)
    total = need + extra_pages
    pool = orc.FifoPagePool(total, len(kv_lens), max(1, max((ln + 15) // 16 for ln in kv_lens)),
                            free_order=workloads.randperm(total, seed))
    for s, ln in enumerate(kv_lens):
        pool.ensure_pages(s, (ln + 15) // 16)
    g = torch.Generator().manual_seed(seed)
    kc = torch.randn(total, 16, hkv, d, generator=g).to(torch.bfloat16)
    vc = torch.randn(total, 16, hkv, d, generator=g).to(torch.bfloat16)
    qo = np.zeros(len(q_lens) + 1, np.int32)
    np.cumsum(q_lens, out=qo[1:])
    kvi, lpl = orc.plan_decode(kv_lens)
    idx = orc.page_indices(pool.block_table, range(len(kv_lens)), kvi)
    q = randn_bf16((int(qo[-1]), hq, d), seed + 1, std=1.5, device=device)
    return q, kc, vc, qo, kvi, idx, lpl


def _run(gpu, q, kc, vc, qo, kvi, idx, lpl, hq, hkv, causal=True, out=None):
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(WS, dtype=torch.uint8, device=gpu))
    w.plan(torch.from_numpy(qo), torch.from_numpy(kvi), torch.from_numpy(idx).to(gpu),
           torch.from_numpy(lpl), num_qo_heads=hq, num_kv_heads=hkv, head_dim_qk=q.shape[-1],
           page_size=16, causal=causal, q_data_type=torch.bfloat16)
    res = w.run(q, (kc.to(gpu), vc.to(gpu)), out=out, return_lse=True)
    torch.cuda.synchronize()
    return res, w


def _check(gpu, q_lens, kv_lens, hq, hkv, seed, causal=True):
    q, kc, vc, qo, kvi, idx, lpl = _case(q_lens, kv_lens, hq, hkv, seed, device=gpu)
    (out, lse), w = _run(gpu, q, kc, vc, qo, kvi, idx, lpl, hq, hkv, causal)
    ref, ref_lse = orc.paged_prefill(u16(q), u16(kc), u16(vc), qo, kvi, idx, lpl, causal=causal)
    assert_attn_close(out.float().cpu().numpy(), ref)
    got_lse = lse.cpu().numpy()
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isneginf(got_lse), ~fin)
    assert np.abs(got_lse[fin] - ref_lse[fin]).max() < LSE_TOL
    return w


def test_prefill_mixed_batch_gqa4(gpu):
    """Chunks at the tail of longer caches, chunks equal to the cache, a
    one-token chunk, partial last pages and query tiles that straddle both
    the chunk end and the causal diagonal."""
    w = _check(gpu, [1, 17, 40, 64, 130, 5, 33], [1, 40, 40, 300, 130, 133, 1000], 32, 8, 30)
    assert w.schedule.tile_tokens == 64 and w.schedule.num_items == 1 + 1 + 1 + 1 + 3 + 1 + 1


@pytest.mark.parametrize("group", [1, 2, 8])
def test_prefill_group_sizes(gpu, group):
    hkv = 4 if group < 8 else 2
    _check(gpu, [70, 3, 200], [70, 90, 333], hkv * group, hkv, 31 + group)


def test_prefill_non_causal(gpu):
    _check(gpu, [50, 8], [50, 300], 32, 8, 33, causal=False)


def test_prefill_edge_cases(gpu):
    """Empty chunks, a request with no pages, and a chunk longer than its
    cache (its first queries see no key: output 0, lse -inf)."""
    _check(gpu, [0, 20, 6, 0, 9], [12, 5, 0, 17, 40], 32, 8, 34)


def test_prefill_random_shapes(gpu):
    """Seeded random batches against the oracle (output and lse): 1-8
    requests, group sizes 1-8, 1-8 KV heads, causal and not; caches of
    0-2500 tokens (some exact page multiples), chunks shorter than, equal to
    or (a few) longer than their cache, empty chunks.  Sizes are scaled down
    so that the oracle's q_len x kv_len x Hq stays under 6e7 per case."""
    rng = np.random.default_rng(47)
    for case in range(20):
        group = int(rng.choice([1, 2, 4, 8]))
        hkv = int(rng.choice([1, 2, 4, 8]))
        hq = hkv * group
        b = int(rng.integers(1, 9))
        kv = np.where(rng.random(b) < 0.2, 16 * rng.integers(0, 40, b), rng.integers(0, 2500, b))
        ql = np.minimum(kv, rng.integers(0, 700, b))
        ql = np.where(rng.random(b) < 0.1, kv + rng.integers(1, 20, b), ql)
        ql = np.where(rng.random(b) < 0.1, 0, ql)
        if ql.sum() == 0:
            ql[0] = 1
        while int((ql * kv).sum()) * hq > 60_000_000:
            kv, ql = (kv + 1) // 2, (ql + 1) // 2
        causal = bool(rng.random() < 0.8)
        q_lens, kv_lens = [int(x) for x in ql], [int(x) for x in kv]
        print(f"prefill random case {case}: G={group} Hkv={hkv} causal={causal} "
              f"q={q_lens} kv={kv_lens}", flush=True)
        _check(gpu, q_lens, kv_lens, hq, hkv, 300 + case, causal=causal)


@pytest.mark.parametrize("q_len,kv_len", [(37, 37), (37, 1000), (130, 1000)])
def test_prefill_nan_past_the_end(gpu, q_len, kv_len):
    """Tokens of the last page past kv_len hold NaN bits; they must not leak.
    At kv_len 1000 (16 key tiles, 8 tokens in the last page) the last tile
    is staged and masked inside the pipelined step, not in the prologue."""
    q, kc, vc, qo, kvi, idx, lpl = _case([q_len], [kv_len], 32, 8, 35, device=gpu)
    last = int(idx[kvi[1] - 1])
    kc[last, kv_len % 16:] = float("nan")
    vc[last, kv_len % 16:] = float("nan")
    (out, lse), _ = _run(gpu, q, kc, vc, qo, kvi, idx, lpl, 32, 8)
    ref, ref_lse = orc.paged_prefill(u16(q), u16(kc), u16(vc), qo, kvi, idx, lpl)
    assert torch.isfinite(out).all()
    assert_attn_close(out.float().cpu().numpy(), ref)
    assert np.abs(lse.cpu().numpy() - ref_lse).max() < LSE_TOL


def test_prefill_missing_pages_are_hidden(gpu):
    """Page ids of -1 and past the cache partway through multi-tile requests
    (and a run of three missing pages) hide their tokens, also on tiles that
    would otherwise be interior; the pages' blocks hold NaN bits, which must
    not leak.  Against the oracle's missing-page semantics; finite output."""
    q_lens, kv_lens = [100, 64, 30, 7], [700, 500, 300, 40]
    q, kc, vc, qo, kvi, idx, lpl = _case(q_lens, kv_lens, 32, 8, 42, device=gpu)
    nb = kc.shape[0]
    hidden = [int(idx[kvi[0] + 5]), int(idx[kvi[2] + 3]), int(idx[kvi[2] + 4]),
              int(idx[kvi[2] + 5])]
    idx = idx.copy()
    idx[kvi[0] + 5] = -1                 # a tile that would be interior
    idx[kvi[1] + 20] = nb + 7            # past the cache, near the chunk
    idx[kvi[2] + 3:kvi[2] + 6] = -1      # three missing pages in a row
    idx[kvi[3]:kvi[4]] = -1              # every page missing: 0 / -inf
    for p in hidden:                     # no page reads these blocks now
        kc[p] = float("nan")
        vc[p] = float("nan")
    (out, lse), _ = _run(gpu, q, kc, vc, qo, kvi, idx, lpl, 32, 8)
    ref, ref_lse = orc.paged_prefill(u16(q), u16(kc), u16(vc), qo, kvi, idx, lpl)
    assert torch.isfinite(out).all()
    assert_attn_close(out.float().cpu().numpy(), ref)
    got_lse = lse.cpu().numpy()
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isneginf(got_lse), ~fin)
    assert np.abs(got_lse[fin] - ref_lse[fin]).max() < LSE_TOL
    assert (out[qo[3]:qo[4]] == 0).all()


def test_prefill_workgroups_chain_many_units(gpu):
    """More (query tile, KV head) units than workgroups, so each persistent
    workgroup runs a list of them: ragged chunks, chunks longer than their
    cache (units that see no key sit between units that do, so a unit after
    them starts cold), missing pages and NaN past the end of partial pages.
    The plan image is read back to show that those chains occur."""
    rng = np.random.default_rng(61)
    q_lens = rng.integers(1, 300, 30).tolist()
    kv_lens = [q + int(rng.integers(0, 500)) for q in q_lens]
    for b in (3, 11, 19):                         # first units see no key
        kv_lens[b] = int(rng.integers(1, max(2, q_lens[b] // 3)))
    q_lens[25], kv_lens[25] = 150, 0              # a request with no pages
    q, kc, vc, qo, kvi, idx, lpl = _case(q_lens, kv_lens, 32, 8, 62, device=gpu)
    idx = idx.copy()
    for b in (4, 8, 13):                          # a missing page mid-request
        if kvi[b + 1] - kvi[b] > 3:
            idx[kvi[b] + 2] = -1
    for b in range(len(q_lens)):                  # NaN bits past kv_len
        if kv_lens[b] % 16:
            last = int(idx[kvi[b + 1] - 1])
            if last >= 0:
                kc[last, kv_lens[b] % 16:] = float("nan")
                vc[last, kv_lens[b] % 16:] = float("nan")
    (out, lse), w = _run(gpu, q, kc, vc, qo, kvi, idx, lpl, 32, 8)
    plan = w._plan_dev.cpu().numpy()
    units = w.schedule.num_items * 8
    wgs = min(256, units)
    table = plan[:2 * wgs].reshape(-1, 2)
    rec = plan[(2 * wgs + 3) // 4 * 4:][:units * 8].reshape(-1, 8)
    assert units > 256 and table[:, 1].max() >= 2
    cold = sum(1 for f, c in table for u in range(f + 1, f + c)
               if rec[u - 1, 6] == 0 and rec[u, 6] > 0)
    assert cold > 0                               # a unit after one with no key tiles
    ref, ref_lse = orc.paged_prefill(u16(q), u16(kc), u16(vc), qo, kvi, idx, lpl)
    assert torch.isfinite(out).all()
    assert_attn_close(out.float().cpu().numpy(), ref)
    got_lse = lse.cpu().numpy()
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isneginf(got_lse), ~fin)
    assert np.abs(got_lse[fin] - ref_lse[fin]).max() < LSE_TOL


def test_prefill_long_continuation(gpu):
    """Two 384-token chunks after 640 and 0 cached tokens (many key tiles)."""
    _check(gpu, [384, 384], [1024, 384], 32, 8, 36)


def test_prefill_one_token_chunks_match_decode_kernel(gpu):
    """A one-token chunk at the tail is a decode step: the MFMA prefill and the
    decode kernel agree."""
    kv_lens = [1, 16, 17, 500, 2000]
    q, kc, vc, qo, kvi, idx, lpl = _case([1] * 5, kv_lens, 32, 8, 37, device=gpu)
    (out, lse), _ = _run(gpu, q, kc, vc, qo, kvi, idx, lpl, 32, 8)
    wd = BatchDecodeWithPagedKVCacheWrapper(torch.empty(128 << 20, dtype=torch.uint8, device=gpu))
    wd.plan(torch.from_numpy(kvi), torch.from_numpy(idx).to(gpu), torch.from_numpy(lpl),
            num_qo_heads=32, num_kv_heads=8, head_dim=128, page_size=16)
    dout, dlse = wd.run(q, (kc.to(gpu), vc.to(gpu)), return_lse=True)
    assert_attn_close(out.float().cpu().numpy(), dout.float().cpu().numpy())
    assert (lse - dlse).abs().max().item() < LSE_TOL


def test_prefill_strided_q_and_out(gpu):
    q, kc, vc, qo, kvi, idx, lpl = _case([45, 20], [100, 20], 32, 8, 38, device=gpu)
    big = torch.zeros(q.shape[0], 48, 128, dtype=torch.bfloat16, device=gpu)
    big[:, 8:40] = q
    qv = big[:, 8:40]
    outbig = torch.full((q.shape[0], 40, 128), 7.0, dtype=torch.bfloat16, device=gpu)
    (out, _), _ = _run(gpu, qv, kc, vc, qo, kvi, idx, lpl, 32, 8, out=outbig[:, 4:36])
    ref, _ = orc.paged_prefill(u16(q), u16(kc), u16(vc), qo, kvi, idx, lpl)
    assert_attn_close(out.float().cpu().numpy(), ref)
    assert (outbig[:, :4] == 7).all() and (outbig[:, 36:] == 7).all()


@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_prefill_writes_only_its_rows(gpu, group):
    """The output rows leave as whole rows, four per store, masked past each
    request's last query: every row and head of a larger buffer outside the
    batch's rows keeps its contents, and every row inside is written (the
    sentinel value 7 appears nowhere in it)."""
    hkv = 8 // group if group < 8 else 1
    hq = hkv * group
    q_lens = [37, 5, 70]       # partial query tiles of every group size
    q, kc, vc, qo, kvi, idx, lpl = _case(q_lens, [300, 40, 70], hq, hkv, 23, device=gpu)
    n = q.shape[0]
    outbig = torch.full((n + 40, hq + 2, 128), 7.0, dtype=torch.bfloat16, device=gpu)
    out = outbig[3:3 + n, 1:1 + hq]
    (res, _), _ = _run(gpu, q, kc, vc, qo, kvi, idx, lpl, hq, hkv, out=out)
    ref, _ = orc.paged_prefill(u16(q), u16(kc), u16(vc), qo, kvi, idx, lpl)
    assert_attn_close(res.float().cpu().numpy(), ref)
    big = outbig.cpu()
    assert (big[:3] == 7).all() and (big[3 + n:] == 7).all()
    assert (big[:, 0] == 7).all() and (big[:, 1 + hq:] == 7).all()
    assert not (big[3:3 + n, 1:1 + hq] == 7).all(dim=-1).any()


def test_prefill_rejects_unsupported(gpu):
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(WS, dtype=torch.uint8, device=gpu))
    i = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="head_dim 128"):
        w.plan(i, torch.tensor([0, 1], dtype=torch.int32), torch.zeros(1, dtype=torch.int32),
               torch.tensor([4], dtype=torch.int32), 32, 8, 64, 16, causal=True)
    with pytest.raises(RuntimeError, match="custom masks"):
        w.plan(i, torch.tensor([0, 1], dtype=torch.int32), torch.zeros(1, dtype=torch.int32),
               torch.tensor([4], dtype=torch.int32), 32, 8, 128, 16, causal=True,
               custom_mask=torch.ones(4, dtype=torch.bool))


def test_cache_continuation_prefill_flow(gpu):
    """The engine's continuation path through PagedKVCache: per chunk,
    ensure_pages -> prepare_prefill_chunk (slots, seq_lens += chunk, plan) ->
    append -> prefill, twice; each chunk attends causally over everything
    cached so far (oracle on the cache's own pages)."""
    from gpu_offloading_amd.kv_cache import PagedKVCache

    cache = PagedKVCache(1, 8, 128, max_seqs=3, max_seq_len=800, num_qo_heads=32,
                         kv_page_budget=120, free_page_order=workloads.randperm(120, 40),
                         device=gpu, workspace_bytes=1 << 20, staging_bytes=1 << 20)
    seqs = [0, 1, 2]
    g = torch.Generator(device=gpu).manual_seed(41)
    for chunk in ([300, 17, 64], [200, 40, 1]):
        for s, c in zip(seqs, chunk):
            cache.ensure_pages(s, (int(cache._seq_lens_cpu[s]) + c + 15) // 16)
        slots = cache.prepare_prefill_chunk(seqs, chunk)
        n = sum(chunk)
        k = torch.randn(n, 8, 128, device=gpu, generator=g).to(torch.bfloat16)
        v = torch.randn(n, 8, 128, device=gpu, generator=g).to(torch.bfloat16)
        q = torch.randn(n, 32, 128, device=gpu, generator=g).to(torch.bfloat16)
        cache.append(0, k, v, slots)
        out, lse = cache.prefill(0, q, return_lse=True)
        torch.cuda.synchronize()
        lens = [int(cache._seq_lens_cpu[s]) for s in seqs]
        kvi, lpl = orc.plan_decode(lens)
        idx = orc.page_indices(cache.block_table.cpu().numpy(), seqs, kvi)
        qo = np.zeros(4, np.int32)
        np.cumsum(chunk, out=qo[1:])
        ref, ref_lse = orc.paged_prefill(u16(q), u16(cache.k_cache[0]), u16(cache.v_cache[0]),
                                         qo, kvi, idx, lpl, causal=True)
        assert_attn_close(out.float().cpu().numpy(), ref)
        assert np.abs(lse.cpu().numpy() - ref_lse).max() < LSE_TOL


@pytest.mark.parametrize("kv_len", [2048, 4096])
def test_prefill_at_the_bench_shape(gpu, kv_len):
    """The benchmark's continuation prefill: 8 requests x 2048-token chunks
    at the tail of 2048 / 4096 cached tokens, Mixtral heads (32 / 8), causal;
    against fp32 torch SDPA with its lower-right causal mask, on the GPU."""
    from torch.nn.attention.bias import causal_lower_right

    q_lens, kv_lens = [2048] * 8, [kv_len] * 8
    q, kc, vc, qo, kvi, idx, lpl = _case(q_lens, kv_lens, 32, 8, 50, device=gpu)
    (out, lse), _ = _run(gpu, q, kc, vc, qo, kvi, idx, lpl, 32, 8)
    kg, vg = kc.to(gpu), vc.to(gpu)
    for b in range(8):
        pages = torch.from_numpy(idx[kvi[b]:kvi[b + 1]].astype(np.int64)).to(gpu)
        k = kg[pages].flatten(0, 1)[:kv_len].float().permute(1, 0, 2)   # [Hkv, n, D]
        v = vg[pages].flatten(0, 1)[:kv_len].float().permute(1, 0, 2)
        k = k.repeat_interleave(4, 0).contiguous()
        v = v.repeat_interleave(4, 0).contiguous()
        qb = q[qo[b]:qo[b + 1]].float().permute(1, 0, 2).contiguous()  # [Hq, 2048, D]
        ref = torch.nn.functional.scaled_dot_product_attention(
            qb, k, v, attn_mask=causal_lower_right(2048, kv_len))
        assert_attn_close(out[qo[b]:qo[b + 1]].float().cpu().numpy(),
                          ref.permute(1, 0, 2).cpu().numpy())


def test_prefill_rejects_a_non_finite_scale(gpu):
    """Hidden keys are masked as -inf scores, which stays exact only for a
    positive, finite scale: run() refuses any other."""
    q, kc, vc, qo, kvi, idx, lpl = _case([5], [20], 32, 8, 39, device=gpu)
    for bad in (float("inf"), 0.0, -1.0):
        w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(WS, dtype=torch.uint8, device=gpu))
        w.plan(torch.from_numpy(qo), torch.from_numpy(kvi), torch.from_numpy(idx).to(gpu),
               torch.from_numpy(lpl), num_qo_heads=32, num_kv_heads=8, head_dim_qk=128,
               page_size=16, causal=True, q_data_type=torch.bfloat16, sm_scale=bad)
        with pytest.raises(RuntimeError, match="positive and finite"):
            w.run(q, (kc.to(gpu), vc.to(gpu)))
