"""GPU parity of paged GQA decode attention: against the fp32 CPU oracle and
an fp32 torch SDPA reference, max-abs-error <= 2e-2 and mean-abs-error <= 2e-3
on the bf16 output."""
import math

import numpy as np
import pytest
import torch

from gpu_offloading_amd import ops, workloads
from gpu_offloading_amd.decode import BatchDecodeWithPagedKVCacheWrapper
from helpers import assert_attn_close, randn_bf16, u16
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu

WS = 128 * 1024 * 1024


def _paged(lens, hkv, d, seed, total_pages=None, device=None, fill_std=1.0):
    """Random paged cache holding sequences of the given lengths in blocks of a
    seeded permuted pool; returns (kc, vc, block_table, indptr, indices, lpl)."""
    need = sum((ln + 15) // 16 for ln in lens)
    total = total_pages or need + 8
    pool = orc.FifoPagePool(total, len(lens), max(1, max((ln + 15) // 16 for ln in lens)),
                            free_order=workloads.randperm(total, seed))
    for s, ln in enumerate(lens):
        pool.ensure_pages(s, (ln + 15) // 16)
    kc = (torch.randn(total, 16, hkv, d, device=device) * fill_std).to(torch.bfloat16)
    vc = torch.randn(total, 16, hkv, d, device=device).to(torch.bfloat16)
    indptr, lpl = orc.plan_decode(lens)
    indices = orc.page_indices(pool.block_table, range(len(lens)), indptr)
    return kc, vc, pool.block_table, indptr, indices, lpl


def _run(gpu, q, kc, vc, indptr, indices, lpl, hq, hkv, d, segs=None, return_lse=True):
    w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(WS, dtype=torch.uint8, device=gpu),
                                           num_segments=segs)
    w.plan(torch.from_numpy(indptr), torch.from_numpy(indices).to(gpu), torch.from_numpy(lpl),
           num_qo_heads=hq, num_kv_heads=hkv, head_dim=d, page_size=16)
    res = w.run(q, (kc, vc), return_lse=return_lse)
    torch.cuda.synchronize()
    return res, w


def _sdpa_ref(q, kc, vc, bt, lens):
    """fp32 torch SDPA (enable_gqa) on the contiguous K/V of each sequence,
    reached through the block table with torch indexing (independent of the
    oracle and of the kernel)."""
    qf = q.float().cpu()
    kc, vc = kc.float().cpu(), vc.float().cpu()
    outs = []
    for b, ln in enumerate(lens):
        pages = torch.from_numpy(bt[b, :(ln + 15) // 16].astype(np.int64))
        K = kc[pages].flatten(0, 1)[:ln].transpose(0, 1).contiguous()  # [Hkv, n, D]
        V = vc[pages].flatten(0, 1)[:ln].transpose(0, 1).contiguous()
        o = torch.nn.functional.scaled_dot_product_attention(
            qf[b][:, None, :], K, V, enable_gqa=True)                      # [Hq, 1, D]
        outs.append(o[:, 0])
    return torch.stack(outs).numpy()


def test_decode_cfg1_vs_oracle_and_sdpa(gpu):
    cfg = workloads.config1(seed=0)
    sh = cfg.shape
    lens = [ln + 1 for ln in cfg.seq_lens]  # the step's own token is attended
    kc, vc, bt, indptr, indices, lpl = _paged(lens, sh.num_kv_heads, sh.head_dim, 1,
                                              total_pages=cfg.total_pages)
    for layer in range(sh.num_layers):
        q = randn_bf16((len(lens), sh.num_qo_heads, sh.head_dim), 50 + layer)
        (out, lse), _ = _run(gpu, q.to(gpu), kc.to(gpu), vc.to(gpu), indptr, indices, lpl,
                             sh.num_qo_heads, sh.num_kv_heads, sh.head_dim)
        ref, ref_lse = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
        assert_attn_close(out.float().cpu().numpy(), ref)
        assert_attn_close(out.float().cpu().numpy(), _sdpa_ref(q, kc, vc, bt, lens))
        assert np.allclose(lse.cpu().numpy(), ref_lse, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("d,lens", [(128, [300, 700, 64, 1000, 90]),   # streaming kernel
                                     (128, [40, 100, 200]),              # small-batch kernel
                                     (64, [300, 700, 64, 1000, 90])])    # register kernel
def test_decode_missing_pages_are_hidden(gpu, d, lens):
    """Page ids of -1 or past the cache hide their tokens (the oracle's
    missing-page semantics); the blocks they used to name hold NaN bits and
    must not leak; a request whose pages are all missing gives 0 / -inf."""
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 8, d, 70 + d + len(lens), device=gpu)
    nb = kc.shape[0]
    idx = indices.copy()
    hidden = [int(idx[indptr[0] + 2]), int(idx[indptr[1] + 1])]
    idx[indptr[0] + 2] = -1
    idx[indptr[1] + 1] = nb + 3
    idx[indptr[-2]:indptr[-1]] = -1
    for p in hidden:
        kc[p] = float("nan")
        vc[p] = float("nan")
    q = randn_bf16((len(lens), 32, d), 71 + d, device=gpu)
    (out, lse), w = _run(gpu, q, kc, vc, indptr, idx, lpl, 32, 8, d)
    ref, ref_lse = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, idx, lpl)
    assert torch.isfinite(out).all()
    assert_attn_close(out.float().cpu().numpy(), ref)
    got = lse.cpu().numpy()
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isneginf(got), ~fin) and fin[:-1].all()
    assert np.abs(got[fin] - ref_lse[fin]).max() < 2e-3
    assert (out[-1] == 0).all()


def test_decode_one_token_context_returns_v0_exactly(gpu):
    lens = [1, 1, 17, 16]  # 17: one token in the second page; 16: full page
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 8, 128, 2)
    q = randn_bf16((4, 32, 128), 3, device=gpu)
    (out, lse), _ = _run(gpu, q, kc.to(gpu), vc.to(gpu), indptr, indices, lpl, 32, 8, 128)
    for b in (0, 1):
        v0 = vc[bt[b, 0], 0]                                   # [Hkv, D]
        assert torch.equal(out[b].cpu(), v0.repeat_interleave(4, dim=0))
    ref, _ = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
    assert_attn_close(out.float().cpu().numpy(), ref)


def test_decode_ignores_nan_in_slots_past_the_end(gpu):
    lens = [5, 33]
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 8, 128, 4)
    # poison every slot past each sequence's end with NaN bit patterns
    for b, ln in enumerate(lens):
        last = bt[b, (ln - 1) // 16]
        kc[last, ln % 16 or 16:] = float("nan")
        vc[last, ln % 16 or 16:] = float("nan")
    q = randn_bf16((2, 32, 128), 5, device=gpu)
    (out, _), _ = _run(gpu, q, kc.to(gpu), vc.to(gpu), indptr, indices, lpl, 32, 8, 128)
    ref, _ = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
    assert_attn_close(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("segs", [1, 3, 8, 41, 1000, None])
def test_decode_segment_counts_agree(gpu, segs):
    """Any split of the batch into segments (one request spread over many
    pieces, many requests in one segment) gives the same attention."""
    lens = [1, 15, 16, 17, 64, 100, 511, 512, 513, 2000]
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 8, 128, 6)
    q = randn_bf16((len(lens), 32, 128), 7, device=gpu)
    (out, lse), w = _run(gpu, q, kc.to(gpu), vc.to(gpu), indptr, indices, lpl, 32, 8, 128,
                         segs=segs)
    if segs is not None:
        total = int(indptr[-1])
        assert w.schedule.num_segments == min(max(segs, (total + 127) // 128), total)
    ref, ref_lse = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
    assert_attn_close(out.float().cpu().numpy(), ref)
    assert np.allclose(lse.cpu().numpy(), ref_lse, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("group,d", [(1, 128), (2, 128), (8, 128), (4, 64), (1, 256), (4, 256), (8, 64)])
def test_decode_group_sizes_and_head_dims(gpu, group, d):
    hkv = 4
    hq = hkv * group
    lens = [3, 77, 300, 1025]
    kc, vc, bt, indptr, indices, lpl = _paged(lens, hkv, d, 8)
    q = randn_bf16((len(lens), hq, d), 9, device=gpu)
    (out, _), _ = _run(gpu, q, kc.to(gpu), vc.to(gpu), indptr, indices, lpl, hq, hkv, d, segs=9)
    ref, _ = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
    assert_attn_close(out.float().cpu().numpy(), ref)


def test_decode_random_shapes(gpu):
    """Seeded random batches against the oracle (output and lse): batch
    sizes 1-48; lengths mixing empty requests, one-page requests, exact
    page multiples and long contexts; group sizes 1-8; head dims 64 / 128 /
    256; 1-8 KV heads; planner-chosen and forced segment counts.  The last
    twelve cases use 8 KV heads of 128 dims (the streaming kernel's
    eight-head workgroups), the last six with requests of at most 16 pages
    (the small-batch kernel).  Lengths are scaled down so that each cache
    stays under 16M elements."""
    rng = np.random.default_rng(31)
    combos = [(1, 128), (2, 128), (4, 128), (8, 128), (1, 64), (4, 64), (8, 64),
              (1, 256), (2, 256), (4, 256)]
    for case in range(36):
        if case < 24:
            group, d = combos[int(rng.integers(len(combos)))]
            hkv = int(rng.choice([1, 2, 4, 8]))
        else:  # the Mixtral-shaped kernels: 8 KV heads of 128 dims
            group, d, hkv = int(rng.choice([1, 2, 4])), 128, 8
        hq = hkv * group
        short = case >= 30  # at most 16 pages per request: the small-batch kernel
        b = int(rng.integers(1, 17 if short else 49))
        kind = rng.random(b)
        lens = np.where(kind < 0.1, 0,
                        np.where(kind < 0.3, rng.integers(1, 17, b),
                                 np.where(kind < 0.5, 16 * rng.integers(1, 17 if short else 20, b),
                                          rng.integers(17, 257 if short else 2500, b))))
        cap = (16 << 20) // (hkv * d)
        while lens.sum() > cap:
            lens = np.where(lens > 16, lens // 2, lens)
        lens = [int(x) for x in lens]
        segs = None if short else [None, None, 1, int(rng.integers(2, 600))][int(rng.integers(4))]
        print(f"decode random case {case}: B={b} G={group} D={d} Hkv={hkv} segs={segs} "
              f"tokens={sum(lens)}", flush=True)
        kc, vc, bt, indptr, indices, lpl = _paged(lens, hkv, d, 100 + case)
        q = randn_bf16((b, hq, d), 200 + case, device=gpu)
        (out, lse), w = _run(gpu, q, kc.to(gpu), vc.to(gpu), indptr, indices, lpl, hq, hkv, d,
                             segs=segs)
        if short and sum(lens):
            assert w.schedule.small_batch == 1
        ref, ref_lse = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
        assert_attn_close(out.float().cpu().numpy(), ref)
        got_lse = lse.cpu().numpy()
        live = [i for i, ln in enumerate(lens) if ln]
        empty = [i for i, ln in enumerate(lens) if not ln]
        if live:
            assert np.allclose(got_lse[live], ref_lse[live], atol=1e-3, rtol=1e-4)
        if empty:
            assert np.isneginf(got_lse[empty]).all()
            assert int(out[empty].abs().sum()) == 0


def test_decode_empty_request_gives_zero_and_neg_inf_lse(gpu):
    lens = [0, 40, 0]
    kc, vc, bt, indptr, indices, lpl = _paged([40], 8, 128, 10)
    indptr = np.array([0, 0, 3, 3], np.int32)
    lpl = np.array([0, 8, 0], np.int32)
    q = randn_bf16((3, 32, 128), 11, device=gpu)
    for segs in (None, 2):
        (out, lse), _ = _run(gpu, q, kc.to(gpu), vc.to(gpu), indptr, indices, lpl, 32, 8, 128,
                             segs=segs)
        assert int(out[0].abs().sum()) == 0 and int(out[2].abs().sum()) == 0
        assert torch.isneginf(lse[0]).all() and torch.isneginf(lse[2]).all()
        ref, _ = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
        assert_attn_close(out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("lens", [[0, 5], [10, 10, 10, 10, 0], [0, 0]])
def test_decode_empty_requests_when_no_request_is_split(gpu, lens):
    """Regression: empty requests beside requests of one piece each (the plan
    has max_partitions 1 and no partials workspace).  The merge launch zeroes
    the empty requests without reading partials; the rest match the oracle."""
    print(f"decode empty-request batch {lens}", flush=True)
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 8, 128, 24)
    q = randn_bf16((len(lens), 32, 128), 25, device=gpu)
    (out, lse), w = _run(gpu, q, kc.to(gpu), vc.to(gpu), indptr, indices, lpl, 32, 8, 128)
    assert w.schedule.max_partitions == 1 and w.schedule.workspace_bytes == 0
    assert w.schedule.num_empty == lens.count(0)
    ref, ref_lse = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
    for b, ln in enumerate(lens):
        if ln == 0:
            assert int(out[b].abs().sum()) == 0
            assert torch.isneginf(lse[b]).all()
    assert_attn_close(out.float().cpu().numpy(), ref)
    live = [b for b, ln in enumerate(lens) if ln]
    if live:
        assert np.allclose(lse[live].cpu().numpy(), ref_lse[live], atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("group", [1, 2, 4, 8])
def test_decode_small_batch_kernel(gpu, group):
    """Small-batch schedules (one workgroup per request and KV head, the
    waves' states merged in LDS): against the oracle and fp32 SDPA, empty
    requests zero / -inf, rows past each request's end poisoned with NaN.
    The last pages hold 1, 3, 4, 5, 8, 13, 15 and 16 rows (p.v stops at the
    first multiple of four past a partial page's rows)."""
    print(f"decode small-batch kernel, group {group}", flush=True)
    hkv = 8 if group <= 4 else 4
    hq = hkv * group
    lens = [129, 1, 0, 256, 17, 16, 100, 21, 24, 45, 47, 3]
    kc, vc, bt, indptr, indices, lpl = _paged(lens, hkv, 128, 26 + group)
    for b, ln in enumerate(lens):
        if ln % 16:
            last = bt[b, (ln - 1) // 16]
            kc[last, ln % 16:] = float("nan")
            vc[last, ln % 16:] = float("nan")
    q = randn_bf16((len(lens), hq, 128), 27, device=gpu)
    (out, lse), w = _run(gpu, q, kc.to(gpu), vc.to(gpu), indptr, indices, lpl, hq, hkv, 128)
    assert w.schedule.small_batch == 1 and w.schedule.workspace_bytes == 0
    ref, ref_lse = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
    got = out.float().cpu().numpy()
    assert_attn_close(got, ref)
    live = [b for b, ln in enumerate(lens) if ln]
    kcf, vcf = kc.clone(), vc.clone()
    kcf[torch.isnan(kcf)] = 0
    vcf[torch.isnan(vcf)] = 0
    assert_attn_close(got[live], _sdpa_ref(q[live], kcf, vcf, bt[live], [lens[b] for b in live]))
    assert np.allclose(lse[live].cpu().numpy(), ref_lse[live], atol=1e-3, rtol=1e-4)
    assert int(out[2].abs().sum()) == 0 and torch.isneginf(lse[2]).all()
    # one-token request: exactly V[0] of its KV heads
    v0 = vc[bt[1, 0], 0]
    assert torch.equal(out[1].cpu(), v0.repeat_interleave(group, dim=0))


def test_decode_batch1_at_the_reference_shape_uses_one_launch(gpu):
    """The reference's published decode shape (one 129-token request,
    Mixtral heads) plans a small-batch schedule and matches the oracle."""
    lens = [129]
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 8, 128, 28)
    q = randn_bf16((1, 32, 128), 29, device=gpu)
    (out, lse), w = _run(gpu, q, kc.to(gpu), vc.to(gpu), indptr, indices, lpl, 32, 8, 128)
    assert w.schedule.small_batch == 1 and w.schedule.max_partitions == 1
    ref, ref_lse = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
    assert_attn_close(out.float().cpu().numpy(), ref)
    assert np.abs(lse.cpu().numpy() - ref_lse).max() < 1e-3


def test_decode_q_view_and_out_buffer(gpu):
    # q as q_buf[:B] of a larger static buffer, out written into a view of a
    # larger [N, Hq*D] buffer (the engine's attn_out_buf), combined KV tensor.
    lens = [40, 200, 1000]
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 8, 128, 12)
    q_buf = randn_bf16((8, 32, 128), 13, device=gpu)
    kv = torch.stack([kc, vc], dim=1).to(gpu)  # [P, 2, 16, H, D]
    w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(WS, dtype=torch.uint8, device=gpu))
    w.plan(torch.from_numpy(indptr), torch.from_numpy(indices), torch.from_numpy(lpl), 32, 8, 128, 16)
    out_buf = torch.zeros(8, 32 * 128, dtype=torch.bfloat16, device=gpu)
    out = w.run(q_buf[:3], kv, out=out_buf[:3].view(3, 32, 128))
    torch.cuda.synchronize()
    assert out.data_ptr() == out_buf.data_ptr()
    ref, _ = orc.paged_decode(u16(q_buf[:3]), u16(kc), u16(vc), indptr, indices, lpl)
    assert_attn_close(out_buf[:3].view(3, 32, 128).float().cpu().numpy(), ref)
    assert int(out_buf[3:].abs().sum()) == 0


def test_decode_cfg2_one_layer(gpu):
    """Config 2 shapes (B=64, ctx U[512, 4096] + the step's token), one layer."""
    cfg = workloads.config2(seed=0)
    lens = [ln + 1 for ln in cfg.seq_lens]
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 8, 128, 14, device=gpu)
    q = randn_bf16((64, 32, 128), 15, device=gpu)
    (out, lse), w = _run(gpu, q, kc, vc, indptr, indices, lpl, 32, 8, 128)
    assert w.schedule.max_partitions > 1  # exercises the split-K merge
    ref, ref_lse = orc.paged_decode(u16(q), u16(kc), u16(vc), indptr, indices, lpl)
    assert_attn_close(out.float().cpu().numpy(), ref)
    assert np.allclose(lse.cpu().numpy(), ref_lse, atol=2e-3, rtol=1e-4)


def test_decode_cfg4_long_context(gpu):
    """Config 4: 16 x 32768 tokens, logits std ~3 (q scaled by 3).  Four of
    the requests (first, last and two inside) are checked against the oracle."""
    cfg = workloads.config4(seed=0)
    lens = cfg.seq_lens
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 8, 128, 16, device=gpu)
    q = randn_bf16((16, 32, 128), 17, std=3.0, device=gpu)
    (out, lse), _ = _run(gpu, q, kc, vc, indptr, indices, lpl, 32, 8, 128)
    kcn, vcn = u16(kc), u16(vc)
    got = out.float().cpu().numpy()
    for b in (0, 5, 10, 15):
        sl = slice(b, b + 1)
        ip = indptr[sl.start:sl.stop + 1] - indptr[b]
        idx = indices[indptr[b]:indptr[b + 1]]
        ref, _ = orc.paged_decode(u16(q[sl]), kcn, vcn, ip, idx, lpl[sl])
        assert_attn_close(got[sl], ref)


def test_decode_cfg5_mha_batch(gpu):
    """Config 5's decode shape: OLMoE attention (MHA, 16 heads), 128
    requests x 2048 tokens from a shuffled 16,384-page pool; six requests
    (first, last and four inside) are checked against the oracle."""
    cfg = workloads.config5(seed=0)
    lens = [ln + 1 for ln in cfg.seq_lens]       # the step's own token is attended
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 16, 128, 18, device=gpu)
    q = randn_bf16((len(lens), 16, 128), 19, device=gpu)
    (out, lse), w = _run(gpu, q, kc, vc, indptr, indices, lpl, 16, 16, 128)
    assert w.schedule.max_partitions > 1
    kcn, vcn = u16(kc), u16(vc)
    got = out.float().cpu().numpy()
    for b in (0, 17, 63, 64, 100, 127):
        sl = slice(b, b + 1)
        ip = indptr[sl.start:sl.stop + 1] - indptr[b]
        idx = indices[indptr[b]:indptr[b + 1]]
        ref, ref_lse = orc.paged_decode(u16(q[sl]), kcn, vcn, ip, idx, lpl[sl])
        assert_attn_close(got[sl], ref)
        assert np.abs(lse[sl].cpu().numpy() - ref_lse).max() < 2e-3


def test_merge_attention_states_matches_oracle(gpu):
    o1 = randn_bf16((5, 32, 128), 20, device=gpu)
    o2 = randn_bf16((5, 32, 128), 21, device=gpu)
    l1 = torch.randn(5, 32, device=gpu) * 4
    l2 = torch.randn(5, 32, device=gpu) * 4
    l2[0, 0] = float("-inf")
    out, lse = ops.merge_attention_states(o1, l1, o2, l2)
    ref_o, ref_l = orc.merge_attention_states(o1.float().cpu().numpy(), l1.cpu().numpy(),
                                              o2.float().cpu().numpy(), l2.cpu().numpy())
    assert_attn_close(out.float().cpu().numpy(), ref_o)
    assert np.allclose(lse.cpu().numpy(), ref_l, atol=1e-5, rtol=1e-5)


def test_decode_split_merge_equals_whole(gpu):
    """Attention over a context split in two halves, merged with
    merge_attention_states, equals attention over the whole context."""
    lens = [700]
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 8, 128, 22)
    q = randn_bf16((1, 32, 128), 23, device=gpu)
    kcg, vcg = kc.to(gpu), vc.to(gpu)
    (whole, _), _ = _run(gpu, q, kcg, vcg, indptr, indices, lpl, 32, 8, 128)
    a_idx, b_idx = indices[:20], indices[20:]
    (o1, l1), _ = _run(gpu, q, kcg, vcg, np.array([0, 20], np.int32), a_idx,
                       np.array([16], np.int32), 32, 8, 128)
    (o2, l2), _ = _run(gpu, q, kcg, vcg, np.array([0, len(b_idx)], np.int32), b_idx,
                       lpl, 32, 8, 128)
    merged, _ = ops.merge_attention_states(o1, l1, o2, l2)
    assert_attn_close(merged.float().cpu().numpy(), whole.float().cpu().numpy())


def test_run_rechecks_caches_after_a_new_plan(gpu):
    """run() checks a cache tensor once per (tensor, plan geometry): a plan
    for other head counts makes the same tensors fail again, and a tensor
    of the wrong geometry is refused even after good ones were accepted."""
    lens = [40, 100]
    kc, vc, bt, indptr, indices, lpl = _paged(lens, 8, 128, 21, device=gpu)
    q = randn_bf16((2, 32, 128), 22, device=gpu)
    out1, w = _run(gpu, q, kc, vc, indptr, indices, lpl, 32, 8, 128, return_lse=False)
    out2 = w.run(q, (kc, vc))                          # cached check, same result
    assert torch.equal(out1, out2)
    w.plan(torch.from_numpy(indptr), torch.from_numpy(indices).to(gpu), torch.from_numpy(lpl),
           num_qo_heads=16, num_kv_heads=4, head_dim=128, page_size=16)
    with pytest.raises(RuntimeError, match="k_cache must be"):
        w.run(randn_bf16((2, 16, 128), 23, device=gpu), (kc, vc))
    w.plan(torch.from_numpy(indptr), torch.from_numpy(indices).to(gpu), torch.from_numpy(lpl),
           num_qo_heads=32, num_kv_heads=8, head_dim=128, page_size=16)
    assert torch.equal(w.run(q, (kc, vc)), out1)
    with pytest.raises(RuntimeError, match="v_cache must be bfloat16"):
        w.run(q, (kc, vc.half()))
