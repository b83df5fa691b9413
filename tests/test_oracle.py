"""Pins of the CPU oracle (oracle/kv_oracle.py), CPU only.

The reference holds no golden vectors, known-answer tests or fixtures for this
path (its arithmetic lives in vLLM 0.17.1 / FlashInfer, absent here), so each
oracle function is pinned by checks that do not retype its formula:
  bf16 conversion     torch's own float32 <-> bfloat16 casts (RNE)
  page pool           the reference allocator's documented FIFO order and
                      errors (moe_engine.py:4231-4297), worked by hand
  slot mapping        identity block tables (static mode, moe_engine.py:504-519)
                      give slot = seq * pages * 16 + pos; injectivity
  plan                hand-worked indptr / last_page_len including len % 16 == 0
  append / gather     element-by-element Python loops; append -> gather identity
  decode attention    torch scaled_dot_product_attention (fp32, enable_gqa) and
                      special cases: one token -> V[0], constant K -> mean(V)
  merge               attention over A ++ B == merge(attn(A), attn(B))
  block gather/scat.  byte images of the blocks; round-trip identity
A deliberately planted mistake in each oracle function fails one of these
(tests at the end plant them in copies of the oracle functions).
"""
import numpy as np
import pytest
import torch

from oracle import kv_oracle as orc


def rand_bf16(rng, shape, std=1.0):
    return orc.f32_to_bf16((rng.standard_normal(shape) * std).astype(np.float32))


# ----------------------------------------------------------------- bf16
def test_bf16_conversions_match_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 1e3,
                        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.0e38, 1e-40,
                                  1.00390625, 1.01171875], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16(x), ref)
    back = torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(orc.bf16_to_f32(ref), back)
    nan = orc.f32_to_bf16(np.array([np.nan], np.float32))
    assert np.isnan(orc.bf16_to_f32(nan)).all()


# ------------------------------------------------------------ page pool
def test_fifo_pool_order_and_errors_by_hand():
    pool = orc.FifoPagePool(6, 3, 4)
    pool.alloc_pages(0, 2)                  # takes 0, 1
    pool.alloc_pages(1, 3)                  # takes 2, 3, 4
    assert pool.block_table[0].tolist() == [0, 1, -1, -1]
    assert pool.block_table[1].tolist() == [2, 3, 4, -1]
    pool.free_seq(0)                        # free list: 5, 0, 1
    assert pool.block_table[0].tolist() == [-1] * 4
    pool.alloc_pages(2, 2)                  # takes 5, 0
    assert pool.block_table[2].tolist() == [5, 0, -1, -1]
    assert (pool.pages_free, pool.pages_in_use) == (1, 5)
    pool.alloc_pages(2, 0)                  # no-op
    pool.alloc_pages(2, -3)                 # no-op
    with pytest.raises(RuntimeError, match="only 1 free pages remain"):
        pool.alloc_pages(0, 2)
    with pytest.raises(RuntimeError, match="max_pages_per_seq"):
        pool.alloc_pages(1, 2)
    pool.ensure_pages(1, 2)                 # already has 3: no-op
    pool.ensure_pages(0, 1)                 # takes 1
    assert pool.block_table[0, 0] == 1 and pool.pages_free == 0
    pool.reset()
    assert pool.pages_free == 6 and (pool.block_table == -1).all()


def test_fifo_pool_custom_free_order():
    pool = orc.FifoPagePool(8, 2, 8, free_order=[7, 2, 5])
    pool.alloc_pages(0, 2)
    assert pool.block_table[0, :2].tolist() == [7, 2]
    assert pool.pages_in_use == 7


# --------------------------------------------------------- slot mapping
def test_slot_mapping_identity_table_closed_form():
    max_seqs, pages = 5, 7
    bt = np.arange(max_seqs * pages, dtype=np.int32).reshape(max_seqs, pages)
    rng = np.random.default_rng(1)
    seqs = rng.integers(0, max_seqs, 200)
    pos = rng.integers(0, pages * 16, 200)
    got = orc.slot_mapping(bt, seqs, pos)
    assert got.dtype == np.int64
    assert np.array_equal(got, seqs * pages * 16 + pos)


def test_slot_mapping_permuted_table_is_injective_and_consistent():
    rng = np.random.default_rng(2)
    bt = rng.permutation(4 * 9).astype(np.int32).reshape(4, 9)
    seqs = np.repeat(np.arange(4), 9 * 16)
    pos = np.tile(np.arange(9 * 16), 4)
    s = orc.slot_mapping(bt, seqs, pos)
    assert len(np.unique(s)) == len(s) == 4 * 9 * 16
    assert np.array_equal(s // 16, bt[seqs, pos // 16]) and np.array_equal(s % 16, pos % 16)


def test_step_slot_mapping_pads_with_minus_one():
    bt = np.arange(3 * 4, dtype=np.int32).reshape(3, 4)
    computed = np.array([5, 0, 17], np.int32)
    slots, pos = orc.step_slot_mapping(bt, [2, 0], [1, 3], computed, graph_n=8)
    assert pos.tolist() == [17, 5, 6, 7, 0, 0, 0, 0]
    assert slots.tolist() == [2 * 64 + 17, 5, 6, 7, -1, -1, -1, -1]


# ----------------------------------------------------------------- plan
def test_plan_decode_by_hand():
    indptr, lpl = orc.plan_decode([1, 16, 17, 0, 32, 33])
    assert indptr.tolist() == [0, 1, 2, 4, 4, 6, 9]
    assert lpl.tolist() == [1, 16, 1, 0, 16, 1]


def test_page_indices_by_hand():
    bt = np.array([[9, 8, 7], [1, 2, 3], [4, 5, 6]], np.int32)
    indptr = np.array([0, 2, 3, 6], np.int32)
    assert orc.page_indices(bt, [2, 0, 1], indptr).tolist() == [4, 5, 9, 1, 2, 3]


# --------------------------------------------------------- append/gather
def _loop_append(key, value, kc, vc, slots):
    nb, bs, h, d = kc.shape
    for i, s in enumerate(slots):
        if s < 0 or s >= nb * bs:
            continue
        for hh in range(h):
            for dd in range(d):
                kc[s // bs, s % bs, hh, dd] = key[i, hh, dd]
                vc[s // bs, s % bs, hh, dd] = value[i, hh, dd]


def test_append_matches_elementwise_loop():
    rng = np.random.default_rng(3)
    nb, h, d, n = 6, 2, 4, 40
    k = rand_bf16(rng, (n + 3, h, d))
    v = rand_bf16(rng, (n + 3, h, d))
    slots = rng.permutation(nb * 16)[:n].astype(np.int64)
    slots[[3, 17]] = -1
    slots[20] = nb * 16 + 5          # out of range: skipped
    kc0 = rand_bf16(rng, (nb, 16, h, d))
    vc0 = rand_bf16(rng, (nb, 16, h, d))
    ek, ev = kc0.copy(), vc0.copy()
    _loop_append(k, v, ek, ev, slots)
    gk, gv = kc0.copy(), vc0.copy()
    orc.reshape_and_cache(k, v, gk, gv, slots)
    assert np.array_equal(gk, ek) and np.array_equal(gv, ev)


def test_append_then_gather_is_identity_with_offsets():
    rng = np.random.default_rng(4)
    lens = [37, 128, 255, 1]
    pool = orc.FifoPagePool(64, 4, 16, free_order=rng.permutation(64).tolist())
    for s, ln in enumerate(lens):
        pool.ensure_pages(s, (ln + 15) // 16)
    seqs = np.concatenate([[s] * ln for s, ln in enumerate(lens)])
    pos = np.concatenate([np.arange(ln) for ln in lens])
    slots = orc.slot_mapping(pool.block_table, seqs, pos)
    k = rand_bf16(rng, (len(slots), 2, 8))
    v = rand_bf16(rng, (len(slots), 2, 8))
    kc = np.zeros((64, 16, 2, 8), np.uint16)
    vc = np.zeros_like(kc)
    orc.reshape_and_cache(k, v, kc, vc, slots)
    gk, gv = orc.gather_kv(kc, vc, pool.block_table, lens)
    assert np.array_equal(gk, k) and np.array_equal(gv, v)
    starts = [3, 100, 0, 0]
    sub = [ln - st for ln, st in zip(lens, starts)]
    gk2, _ = orc.gather_kv(kc, vc, pool.block_table, sub, starts)
    cu = np.concatenate([[0], np.cumsum(lens)])
    exp = np.concatenate([k[cu[b] + starts[b]:cu[b + 1]] for b in range(4)])
    assert np.array_equal(gk2, exp)


# ------------------------------------------------------------- decode
def _sdpa(q_bits, kc, vc, bt, lens):
    q = torch.from_numpy(orc.bf16_to_f32(q_bits))
    K = torch.from_numpy(orc.bf16_to_f32(kc))
    V = torch.from_numpy(orc.bf16_to_f32(vc))
    outs = []
    for b, ln in enumerate(lens):
        pages = torch.from_numpy(bt[b, :(ln + 15) // 16].astype(np.int64))
        Kb = K[pages].flatten(0, 1)[:ln].transpose(0, 1).contiguous()
        Vb = V[pages].flatten(0, 1)[:ln].transpose(0, 1).contiguous()
        o = torch.nn.functional.scaled_dot_product_attention(q[b][:, None], Kb, Vb, enable_gqa=True)
        outs.append(o[:, 0])
    return torch.stack(outs).numpy()


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (16, 16, 64), (8, 2, 32)])
def test_paged_decode_matches_torch_sdpa(hq, hkv, d):
    rng = np.random.default_rng(5)
    lens = [1, 15, 16, 17, 100, 300]
    pool = orc.FifoPagePool(64, len(lens), 32, free_order=rng.permutation(64).tolist())
    for s, ln in enumerate(lens):
        pool.ensure_pages(s, (ln + 15) // 16)
    kc = rand_bf16(rng, (64, 16, hkv, d))
    vc = rand_bf16(rng, (64, 16, hkv, d))
    q = rand_bf16(rng, (len(lens), hq, d), std=2.0)
    indptr, lpl = orc.plan_decode(lens)
    idx = orc.page_indices(pool.block_table, range(len(lens)), indptr)
    out, lse = orc.paged_decode(q, kc, vc, indptr, idx, lpl)
    ref = _sdpa(q, kc, vc, pool.block_table, lens)
    assert np.abs(out - ref).max() < 2e-5
    # lse against torch.logsumexp of the scaled logits, one request
    b, ln = 4, lens[4]
    K = orc.bf16_to_f32(kc)[pool.block_table[b, :(ln + 15) // 16]].reshape(-1, hkv, d)[:ln]
    qf = orc.bf16_to_f32(q)[b]
    g = hq // hkv
    logits = np.stack([qf[h] @ K[:, h // g].T for h in range(hq)]) / np.sqrt(d)
    assert np.allclose(lse[b], torch.logsumexp(torch.from_numpy(logits), -1).numpy(), atol=1e-5)


def test_paged_decode_special_cases():
    rng = np.random.default_rng(6)
    kc = rand_bf16(rng, (4, 16, 2, 16))
    vc = rand_bf16(rng, (4, 16, 2, 16))
    q = rand_bf16(rng, (2, 4, 16))
    # one-token context: the output is V[0] of the mapped kv head
    out, lse = orc.paged_decode(q, kc, vc, np.array([0, 1, 2], np.int32),
                                np.array([3, 1], np.int32), np.array([1, 1], np.int32))
    for b, page in enumerate([3, 1]):
        exp = orc.bf16_to_f32(vc[page, 0])[[0, 0, 1, 1]]
        assert np.array_equal(out[b], exp)
    # constant K: uniform weights, the output is the mean of V over the context
    kc2 = np.full_like(kc, orc.f32_to_bf16(np.float32(0.5)))
    out, lse = orc.paged_decode(q[:1], kc2, vc, np.array([0, 2], np.int32),
                                np.array([2, 0], np.int32), np.array([5], np.int32))
    V = orc.bf16_to_f32(vc[[2, 0]]).reshape(-1, 2, 16)[:21]
    assert np.allclose(out[0], V.mean(0)[[0, 0, 1, 1]], atol=1e-6)
    # empty request: zero output, lse -inf
    out, lse = orc.paged_decode(q[:1], kc, vc, np.array([0, 0], np.int32), np.zeros(0, np.int32),
                                np.array([0], np.int32))
    assert (out == 0).all() and np.isneginf(lse).all()


def test_merge_of_split_context_equals_whole():
    rng = np.random.default_rng(7)
    kc = rand_bf16(rng, (16, 16, 2, 32))
    vc = rand_bf16(rng, (16, 16, 2, 32))
    q = rand_bf16(rng, (1, 8, 32), std=3.0)
    pages = rng.permutation(16)[:10].astype(np.int32)
    whole, lw = orc.paged_decode(q, kc, vc, np.array([0, 10], np.int32), pages, np.array([7], np.int32))
    o1, l1 = orc.paged_decode(q, kc, vc, np.array([0, 4], np.int32), pages[:4], np.array([16], np.int32))
    o2, l2 = orc.paged_decode(q, kc, vc, np.array([0, 6], np.int32), pages[4:], np.array([7], np.int32))
    m, lm = orc.merge_attention_states(o1, l1, o2, l2)
    assert np.allclose(m, whole, atol=1e-5) and np.allclose(lm, lw, atol=1e-5)
    # merging with an empty state (lse -inf) is the identity
    m2, l2m = orc.merge_attention_states(o1, l1, np.zeros_like(o1), np.full_like(l1, -np.inf))
    assert np.allclose(m2, o1) and np.allclose(l2m, l1)


# -------------------------------------------------------------- blocks
def test_gather_scatter_blocks_byte_images():
    rng = np.random.default_rng(8)
    kc = rand_bf16(rng, (10, 16, 2, 8))
    vc = rand_bf16(rng, (10, 16, 2, 8))
    ids = np.array([7, 2, 9], np.int32)
    st = orc.gather_blocks(kc, vc, ids)
    assert st.shape == (3, 2, 16 * 2 * 8 * 2) and st.dtype == np.uint8
    for i, b in enumerate(ids):
        assert st[i, 0].tobytes() == kc[b].tobytes() and st[i, 1].tobytes() == vc[b].tobytes()
    k2, v2 = np.zeros_like(kc), np.zeros_like(vc)
    orc.scatter_blocks(st, [0, 5, 1], k2, v2)
    assert np.array_equal(k2[[0, 5, 1]], kc[ids]) and np.array_equal(v2[[0, 5, 1]], vc[ids])
    assert (k2[[2, 3, 4, 6, 7, 8, 9]] == 0).all()


# ----------------------------------------------- planted mistakes fail
def test_planted_mistakes_are_caught():
    """Copies of oracle functions with a typical slip (wrong GQA head map,
    missing scale, off-by-one last page) disagree with the pins above."""
    rng = np.random.default_rng(9)
    lens = [20, 33]
    pool = orc.FifoPagePool(16, 2, 8, free_order=rng.permutation(16).tolist())
    for s, ln in enumerate(lens):
        pool.ensure_pages(s, (ln + 15) // 16)
    kc = rand_bf16(rng, (16, 16, 2, 16))
    vc = rand_bf16(rng, (16, 16, 2, 16))
    q = rand_bf16(rng, (2, 4, 16), std=2.0)
    indptr, lpl = orc.plan_decode(lens)
    idx = orc.page_indices(pool.block_table, [0, 1], indptr)
    ref = _sdpa(q, kc, vc, pool.block_table, lens)

    def bad_decode(headmap=None, scale=None, lpl_shift=0):
        qf = orc.bf16_to_f32(q)
        out = np.zeros_like(qf)
        for b in range(2):
            pages = idx[indptr[b]:indptr[b + 1]]
            n = (len(pages) - 1) * 16 + int(lpl[b]) + lpl_shift
            K = orc.bf16_to_f32(kc[pages].reshape(-1, 2, 16)[:n])
            V = orc.bf16_to_f32(vc[pages].reshape(-1, 2, 16)[:n])
            for h in range(4):
                kh = headmap(h) if headmap else h // 2
                s = K[:, kh] @ qf[b, h] * (scale if scale else 1 / 4.0)
                p = np.exp(s - s.max())
                out[b, h] = p @ V[:, kh] / p.sum()
        return out

    assert np.abs(bad_decode() - ref).max() < 2e-5                        # the correct form
    assert np.abs(bad_decode(headmap=lambda h: h % 2) - ref).max() > 1e-2  # interleaved map
    assert np.abs(bad_decode(scale=1.0) - ref).max() > 1e-2                # no 1/sqrt(d)
    assert np.abs(bad_decode(lpl_shift=-1) - ref).max() > 1e-3             # drops last token


# ------------------------------------------------------------ paged prefill
def _prefill_case(rng, q_lens, kv_lens, hq, hkv, d, nblocks=96):
    pool = orc.FifoPagePool(nblocks, len(kv_lens), 64, free_order=rng.permutation(nblocks).tolist())
    for s, ln in enumerate(kv_lens):
        pool.ensure_pages(s, (ln + 15) // 16)
    kc = rand_bf16(rng, (nblocks, 16, hkv, d))
    vc = rand_bf16(rng, (nblocks, 16, hkv, d))
    qo = np.zeros(len(q_lens) + 1, np.int32)
    np.cumsum(q_lens, out=qo[1:])
    q = rand_bf16(rng, (int(qo[-1]), hq, d), std=2.0)
    kv_indptr, lpl = orc.plan_decode(kv_lens)
    idx = orc.page_indices(pool.block_table, range(len(kv_lens)), kv_indptr)
    return q, kc, vc, qo, kv_indptr, idx, lpl, pool.block_table


def _sdpa_prefill(q_bits, kc, vc, qo, bt, kv_lens, mask_fn):
    """torch SDPA per request, fp32, with a torch-built attention bias."""
    q = torch.from_numpy(orc.bf16_to_f32(q_bits))
    K = torch.from_numpy(orc.bf16_to_f32(kc))
    V = torch.from_numpy(orc.bf16_to_f32(vc))
    outs = []
    for b, ln in enumerate(kv_lens):
        qb = q[qo[b]:qo[b + 1]].transpose(0, 1).contiguous()          # [Hq, q_len, D]
        pages = torch.from_numpy(bt[b, :(ln + 15) // 16].astype(np.int64))
        Kb = K[pages].flatten(0, 1)[:ln].transpose(0, 1).contiguous()  # [Hkv, n, D]
        Vb = V[pages].flatten(0, 1)[:ln].transpose(0, 1).contiguous()
        o = torch.nn.functional.scaled_dot_product_attention(
            qb[None], Kb[None], Vb[None], attn_mask=mask_fn(qb.shape[1], ln), enable_gqa=True)
        outs.append(o[0].transpose(0, 1))
    return torch.cat(outs).numpy()


@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (8, 8, 64), (16, 2, 32)])
def test_paged_prefill_matches_sdpa_lower_right_causal(hq, hkv, d):
    """Chunks at the tail of the cache: torch's lower-right causal bias is
    exactly 'query i sees keys j <= i + kv_len - q_len'."""
    from torch.nn.attention.bias import causal_lower_right

    rng = np.random.default_rng(21)
    q_lens, kv_lens = [1, 17, 40, 64, 5], [1, 40, 40, 300, 133]
    q, kc, vc, qo, kvi, idx, lpl, bt = _prefill_case(rng, q_lens, kv_lens, hq, hkv, d)
    out, lse = orc.paged_prefill(q, kc, vc, qo, kvi, idx, lpl, causal=True)
    ref = _sdpa_prefill(q, kc, vc, qo, bt, kv_lens, lambda m, n: causal_lower_right(m, n))
    assert np.abs(out - ref).max() < 3e-5
    # non-causal: no mask at all
    out_nc, _ = orc.paged_prefill(q, kc, vc, qo, kvi, idx, lpl, causal=False)
    ref_nc = _sdpa_prefill(q, kc, vc, qo, bt, kv_lens, lambda m, n: None)
    assert np.abs(out_nc - ref_nc).max() < 3e-5
    # a planted mistake -- the mask aligned to the start of the cache -- is caught
    from torch.nn.attention.bias import causal_upper_left
    wrong = _sdpa_prefill(q, kc, vc, qo, bt, kv_lens, lambda m, n: causal_upper_left(m, n))
    assert np.abs(out - wrong).max() > 1e-2
    # lse of the last row of request 3 (it sees every key) = logsumexp of its logits
    b, row = 3, int(qo[4]) - 1
    K = orc.bf16_to_f32(kc)[bt[b, :(kv_lens[b] + 15) // 16]].reshape(-1, hkv, d)[:kv_lens[b]]
    qf = orc.bf16_to_f32(q)[row]
    g = hq // hkv
    logits = np.stack([qf[h] @ K[:, h // g].T for h in range(hq)]) / np.sqrt(d)
    assert np.allclose(lse[row], torch.logsumexp(torch.from_numpy(logits), -1).numpy(), atol=1e-5)


def test_paged_prefill_one_token_chunks_equal_decode():
    """A one-token chunk at the tail is a decode step over the whole cache."""
    rng = np.random.default_rng(22)
    kv_lens = [1, 16, 17, 250]
    q, kc, vc, qo, kvi, idx, lpl, bt = _prefill_case(rng, [1] * 4, kv_lens, 32, 8, 128)
    out, lse = orc.paged_prefill(q, kc, vc, qo, kvi, idx, lpl, causal=True)
    dec, dlse = orc.paged_decode(q, kc, vc, kvi, idx, lpl)
    assert np.abs(out - dec).max() < 1e-5 and np.abs(lse - dlse).max() < 1e-5


def test_missing_pages_are_hidden():
    """A page id outside [0, num_blocks) (-1, or past the cache) hides its
    tokens: decode and prefill equal torch SDPA over the same keys with those
    tokens masked out by an explicit boolean mask (causal and lower-right for
    prefill); a request whose pages are all missing gives 0 / -inf.  A planted
    mistake -- numpy's wrap-around of -1 to the last block, unmasked -- is
    caught."""
    from torch.nn.attention.bias import causal_lower_right

    rng = np.random.default_rng(26)
    nb, hq, hkv, d = 96, 8, 2, 32
    kv_lens, q_lens = [100, 70, 40], [30, 5, 40]
    q, kc, vc, qo, kvi, idx, lpl, bt = _prefill_case(rng, q_lens, kv_lens, hq, hkv, d, nb)
    bad = idx.copy()
    bad[kvi[0] + 2] = -1            # request 0: page 2 unallocated
    bad[kvi[1] + 4] = nb + 5        # request 1: its last page past the cache
    bad[kvi[2]:kvi[3]] = -1         # request 2: every page missing
    Kf, Vf = torch.from_numpy(orc.bf16_to_f32(kc)), torch.from_numpy(orc.bf16_to_f32(vc))
    qf = torch.from_numpy(orc.bf16_to_f32(q))

    def masked_sdpa(b, rows, causal):
        ln = kv_lens[b]
        pages = bad[kvi[b]:kvi[b + 1]].astype(np.int64)
        ok = (pages >= 0) & (pages < nb)
        present = torch.from_numpy(np.repeat(ok, 16)[:ln])
        safe = torch.from_numpy(np.where(ok, pages, 0))
        Kb = Kf[safe].flatten(0, 1)[:ln].transpose(0, 1).contiguous()
        Vb = Vf[safe].flatten(0, 1)[:ln].transpose(0, 1).contiguous()
        qb = rows.transpose(0, 1).contiguous()                       # [Hq, m, D]
        mask = present[None, :].expand(qb.shape[1], ln)
        if causal:
            mask = mask & causal_lower_right(qb.shape[1], ln)._materialize()
        o = torch.nn.functional.scaled_dot_product_attention(
            qb[None], Kb[None], Vb[None], attn_mask=mask, enable_gqa=True)
        return o[0].transpose(0, 1).numpy()

    out, lse = orc.paged_prefill(q, kc, vc, qo, kvi, bad, lpl, causal=True)
    for b in (0, 1):
        ref = masked_sdpa(b, qf[qo[b]:qo[b + 1]], causal=True)
        assert np.abs(out[qo[b]:qo[b + 1]] - ref).max() < 3e-5
    assert (out[qo[2]:qo[3]] == 0).all() and np.isneginf(lse[qo[2]:qo[3]]).all()
    # decode: the last query row of each request, over the whole cache
    dq = np.stack([q[qo[b + 1] - 1] for b in range(3)])
    dout, dlse = orc.paged_decode(dq, kc, vc, kvi, bad, lpl)
    for b in (0, 1):
        ref = masked_sdpa(b, qf[qo[b + 1] - 1:qo[b + 1]], causal=False)[0]
        assert np.abs(dout[b] - ref).max() < 3e-5
    assert (dout[2] == 0).all() and np.isneginf(dlse[2]).all()
    # the planted mistake: index with the raw ids (-1 wraps to block nb-1)
    K = orc.bf16_to_f32(kc)[bad[kvi[0]:kvi[1]]].reshape(-1, hkv, d)[:kv_lens[0]]
    V = orc.bf16_to_f32(vc)[bad[kvi[0]:kvi[1]]].reshape(-1, hkv, d)[:kv_lens[0]]
    s = K[:, 0] @ orc.bf16_to_f32(dq)[0, 0] / np.sqrt(d)
    p = np.exp(s - s.max())
    assert np.abs(p @ V[:, 0] / p.sum() - dout[0, 0]).max() > 1e-3


def test_paged_prefill_edge_cases():
    rng = np.random.default_rng(23)
    q, kc, vc, qo, kvi, idx, lpl, bt = _prefill_case(rng, [3, 0, 4], [2, 5, 4], 4, 2, 16)
    out, lse = orc.paged_prefill(q, kc, vc, qo, kvi, idx, lpl, causal=True)
    # request 0: 3 queries over 2 keys -- query 0 sees nothing (0, -inf),
    # query 1 sees key 0 only (= V[0] of its kv head), query 2 sees both
    V = orc.bf16_to_f32(vc)[bt[0, 0], :2]                      # [2, Hkv, D]
    assert (out[0] == 0).all() and np.isneginf(lse[0]).all()
    assert np.array_equal(out[1], V[0][[0, 0, 1, 1]])
    assert np.isfinite(lse[2]).all()
    # request 2: q_len == kv_len -- plain causal, query 0 sees key 0 only
    V2 = orc.bf16_to_f32(vc)[bt[2, 0], :4]
    assert np.array_equal(out[3], V2[0][[0, 0, 1, 1]])


# ------------------------------------------------- x-packed layout (f3)
def test_xpacked_append_is_a_relayout_of_the_flat_append():
    """Appending the same tokens to both layouts: the x-packed caches, read
    through the closed-form transpose, equal the flat NHD caches; and a
    hand-placed element lands where vLLM's layout puts it."""
    rng = np.random.default_rng(50)
    H, D, nb = 3, 16, 6
    n = 40
    key = rng.integers(0, 1 << 16, (n, H, D), dtype=np.uint16)
    val = rng.integers(0, 1 << 16, (n, H, D), dtype=np.uint16)
    slots = rng.permutation(nb * 16)[:n].astype(np.int64)
    slots[3] = -1
    kx = np.zeros((nb, H, D // 8, 16, 8), np.uint16)
    vx = np.zeros((nb, H, D, 16), np.uint16)
    orc.reshape_and_cache_xpacked(key, val, kx, vx, slots)
    kf = np.zeros((nb, 16, H, D), np.uint16)
    vf = np.zeros_like(kf)
    orc.reshape_and_cache(key, val, kf, vf, slots)
    kn, vn = orc.xpacked_to_nhd(kx, vx)
    assert np.array_equal(kn, kf) and np.array_equal(vn, vf)
    i, h, d = 7, 2, 13
    blk, off = divmod(int(slots[i]), 16)
    assert kx[blk, h, d // 8, off, d % 8] == key[i, h, d]
    assert vx[blk, h, d, off] == val[i, h, d]


@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 2)])
def test_xpacked_attention_matches_sdpa_and_partitions_merge(hq, hkv):
    rng = np.random.default_rng(51)
    D, nb = 128, 160
    lens = [1, 300, 1100, 512, 17]
    bt = np.full((len(lens), 70), -1, np.int32)
    perm = rng.permutation(nb)
    at = 0
    for b, n in enumerate(lens):
        k = (n + 15) // 16
        bt[b, :k] = perm[at:at + k]
        at += k
    f16 = lambda a: a.astype(np.float16).view(np.uint16)
    kx = f16(rng.standard_normal((nb, hkv, D // 8, 16, 8)))
    vx = f16(rng.standard_normal((nb, hkv, D, 16)))
    q = f16(rng.standard_normal((len(lens), hq, D)))
    scale = 1 / np.sqrt(D)
    out, ml, es, tmp = orc.paged_attention_xpacked(q, kx, vx, bt, np.array(lens), scale)
    # torch SDPA on the same fp16 values (fp32 math), through the transpose
    kn, vn = orc.xpacked_to_nhd(kx, vx)
    K = torch.from_numpy(orc.elem_to_f32(kn, "fp16"))
    V = torch.from_numpy(orc.elem_to_f32(vn, "fp16"))
    qf = torch.from_numpy(orc.elem_to_f32(q, "fp16"))
    for b, n in enumerate(lens):
        pages = torch.from_numpy(bt[b, :(n + 15) // 16].astype(np.int64))
        Kb = K[pages].flatten(0, 1)[:n].transpose(0, 1).contiguous()
        Vb = V[pages].flatten(0, 1)[:n].transpose(0, 1).contiguous()
        ref = torch.nn.functional.scaled_dot_product_attention(qf[b][:, None], Kb, Vb,
                                                               enable_gqa=True)[:, 0]
        assert np.abs(out[b] - ref.numpy()).max() < 3e-5
    # vLLM's v2 reduce of the partitions gives the whole-sequence answer
    for b, n in enumerate(lens):
        P = (n + 511) // 512
        M = ml[b, :, :P].max(axis=1, keepdims=True)
        w = es[b, :, :P] * np.exp(ml[b, :, :P] - M)
        red = (w[..., None] * tmp[b, :, :P]).sum(1) / w.sum(1, keepdims=True)
        assert np.abs(red - out[b]).max() < 3e-5
        assert np.isneginf(ml[b, :, P:]).all()
    # a planted mistake -- the key's 16-byte chunks read in reverse order -- is caught
    wrong, *_ = orc.paged_attention_xpacked(q, np.ascontiguousarray(kx[:, :, ::-1]), vx, bt,
                                            np.array(lens), scale)
    assert np.abs(wrong - out).max() > 1e-2


# --------------------------------------- torch-CPU restatement (baseline)
def test_torch_cpu_restatement_equals_the_oracle():
    """oracle/torch_cpu.py (the multi-core CPU baseline bench.py times) gives
    the oracle's results on the same inputs: bit for bit for append, gather
    and block swap, within float32 rounding for decode."""
    from oracle import torch_cpu as tc

    def t16(a):
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)

    rng = np.random.default_rng(40)
    P, H, Hq, D = 40, 4, 16, 128
    lens = [1, 16, 17, 100, 0, 255]
    pool = orc.FifoPagePool(P, len(lens), 16, free_order=rng.permutation(P).tolist())
    for s, ln in enumerate(lens):
        pool.ensure_pages(s, (ln + 15) // 16)
    kc, vc = rand_bf16(rng, (P, 16, H, D)), rand_bf16(rng, (P, 16, H, D))
    n = sum(lens)
    k, v = rand_bf16(rng, (n + 3, H, D)), rand_bf16(rng, (n + 3, H, D))
    step, _ = orc.step_slot_mapping(pool.block_table, range(len(lens)), lens,
                                    np.zeros(len(lens), np.int64), n)
    slots = np.concatenate([step, [-1, P * 16, -5]]).astype(np.int64)
    # append
    ek, ev = kc.copy(), vc.copy()
    orc.reshape_and_cache(k, v, ek, ev, slots)
    gk, gv = t16(kc.copy()), t16(vc.copy())
    tc.reshape_and_cache(t16(k), t16(v), gk, gv, torch.from_numpy(slots))
    assert np.array_equal(gk.view(torch.int16).numpy().view(np.uint16), ek)
    assert np.array_equal(gv.view(torch.int16).numpy().view(np.uint16), ev)
    # gather
    ok, ov = orc.gather_kv(ek, ev, pool.block_table, lens)
    tk, tv = tc.gather_kv(gk, gv, torch.from_numpy(pool.block_table), lens)
    assert np.array_equal(tk.view(torch.int16).numpy().view(np.uint16), ok)
    assert np.array_equal(tv.view(torch.int16).numpy().view(np.uint16), ov)
    # decode
    q = rand_bf16(rng, (len(lens), Hq, D))
    indptr, lpl = orc.plan_decode(lens)
    idx = orc.page_indices(pool.block_table, range(len(lens)), indptr)
    ro, rl = orc.paged_decode(q, ek, ev, indptr, idx, lpl)
    to, tl = tc.paged_decode(t16(q), gk, gv, torch.from_numpy(indptr), torch.from_numpy(idx),
                             torch.from_numpy(lpl))
    assert np.allclose(to.numpy(), ro, atol=2e-6, rtol=1e-5)
    assert np.allclose(tl.numpy(), rl, atol=2e-6, rtol=1e-5)
    # swap: block images and the round trip
    ids = np.array([idx[3], idx[0], idx[7]], np.int32)
    img = orc.gather_blocks(ek, ev, ids)
    timg = tc.gather_blocks(gk, gv, torch.from_numpy(ids))
    assert np.array_equal(timg.numpy(), img)
    zk, zv = torch.zeros_like(gk), torch.zeros_like(gv)
    tc.scatter_blocks(timg, torch.from_numpy(ids), zk, zv)
    assert torch.equal(zk[ids.astype(np.int64)], gk[ids.astype(np.int64)])
    assert torch.equal(zv[ids.astype(np.int64)], gv[ids.astype(np.int64)])
