"""GPU parity on a cache larger than 4 GiB (one layer, 72,000 pages of the
combined [P, 2, 16, 8, 128] bf16 layout = 4.4 GiB): blocks past byte offset
2^32 are appended (bit-exact), gathered (bit-exact), swapped out and back
(bit-exact), and attended by decode and continuation prefill (oracle
tolerance), so every kernel's block addressing is checked with 64-bit
offsets.  The oracle sees only the touched pages (indices remapped)."""
import numpy as np
import pytest
import torch

from gpu_offloading_amd import ops
from gpu_offloading_amd.decode import BatchDecodeWithPagedKVCacheWrapper
from gpu_offloading_amd.prefill import BatchPrefillWithPagedKVCacheWrapper
from helpers import assert_attn_close, randn_bf16, u16
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu

P, H, HQ, D = 72_000, 8, 32, 128


@pytest.fixture(scope="module")
def big(gpu):
    kv = torch.empty(P, 2, 16, H, D, dtype=torch.bfloat16, device=gpu)
    assert kv.numel() * 2 > 1 << 32
    yield kv
    del kv
    torch.cuda.empty_cache()


def _pages(lens, rng):
    """Page ids for each request, most of them past byte offset 2^32."""
    need = sum((ln + 15) // 16 for ln in lens)
    hi = rng.choice(np.arange(66_000, P - 1), size=need - 3, replace=False)
    ids = np.concatenate([[P - 1, 0, 40_000], hi]).astype(np.int32)
    out, at = [], 0
    for ln in lens:
        n = (ln + 15) // 16
        out.append(ids[at:at + n])
        at += n
    return out


def test_append_gather_decode_prefill_swap_past_4gib(gpu, big):
    rng = np.random.default_rng(5)
    kc, vc = big[:, 0], big[:, 1]
    lens = [300, 17, 1000, 64]
    pages = _pages(lens, rng)
    n = sum(lens)
    # append every token of every request (slots through the page lists)
    slots = np.concatenate([pg[np.arange(ln) // 16].astype(np.int64) * 16 + np.arange(ln) % 16
                            for pg, ln in zip(pages, lens)])
    k = randn_bf16((n, H, D), 11)
    v = randn_bf16((n, H, D), 12)
    ops.reshape_and_cache_flash(k.to(gpu), v.to(gpu), kc, vc, torch.from_numpy(slots).to(gpu),
                                "auto", None, None)
    sl = torch.from_numpy(slots).to(gpu)
    pg_, off_ = sl // 16, sl % 16
    assert torch.equal(kc[pg_, off_].cpu(), k) and torch.equal(vc[pg_, off_].cpu(), v)

    # gather back through a block table
    width = max(len(p) for p in pages)
    bt = np.full((len(lens), width), -1, np.int32)
    for i, pg in enumerate(pages):
        bt[i, :len(pg)] = pg
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    gk, gv = ops.gather_kv(kc, vc, torch.from_numpy(bt).to(gpu), torch.from_numpy(cu).to(gpu),
                           max(lens))
    assert torch.equal(gk.cpu(), k) and torch.equal(gv.cpu(), v)

    # the touched pages, remapped to 0..m-1 for the oracle
    all_pages = np.concatenate(pages)
    sub_k = u16(kc[torch.from_numpy(all_pages).long().to(gpu)])
    sub_v = u16(vc[torch.from_numpy(all_pages).long().to(gpu)])
    remap = np.arange(len(all_pages), dtype=np.int32)
    indptr, lpl = orc.plan_decode(lens)

    # decode
    q = randn_bf16((len(lens), HQ, D), 13)
    w = BatchDecodeWithPagedKVCacheWrapper(torch.empty(1 << 24, dtype=torch.uint8, device=gpu))
    w.plan(torch.from_numpy(indptr), torch.from_numpy(all_pages).to(gpu), torch.from_numpy(lpl),
           num_qo_heads=HQ, num_kv_heads=H, head_dim=D, page_size=16)
    out = w.run(q.to(gpu), (kc, vc))
    ref, _ = orc.paged_decode(u16(q), sub_k, sub_v, indptr, remap, lpl)
    assert_attn_close(out.float().cpu().numpy(), ref)

    # continuation prefill: the last 40 tokens of each request as queries
    chunk = [min(40, ln) for ln in lens]
    qo = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    qp = randn_bf16((int(qo[-1]), HQ, D), 14)
    pw = BatchPrefillWithPagedKVCacheWrapper(torch.empty(16, dtype=torch.uint8, device=gpu))
    pw.plan(torch.from_numpy(qo), torch.from_numpy(indptr), torch.from_numpy(all_pages).to(gpu),
            torch.from_numpy(lpl), num_qo_heads=HQ, num_kv_heads=H, head_dim_qk=D,
            page_size=16, causal=True)
    pout = pw.run(qp.to(gpu), (kc, vc))
    pref, _ = orc.paged_prefill(u16(qp), sub_k, sub_v, qo, indptr, remap, lpl)
    assert_attn_close(pout.float().cpu().numpy(), pref)

    # swap the high pages out, clobber them, swap them back
    ids = torch.from_numpy(all_pages).to(gpu)
    bb = ops.block_bytes(kc)
    host = torch.empty(len(all_pages) * 2 * bb, dtype=torch.uint8, pin_memory=True)
    staging = torch.empty(7 * 2 * bb, dtype=torch.uint8, device=gpu)
    ops.swap_out_blocks([kc], [vc], ids, host, staging)
    torch.cuda.synchronize()
    assert np.array_equal(host.numpy(), orc.gather_blocks(sub_k, sub_v, remap).ravel())
    kc[ids.long()] = 0
    vc[ids.long()] = 0
    ops.swap_in_blocks(host, ids, [kc], [vc], staging)
    torch.cuda.synchronize()
    assert np.array_equal(u16(kc[ids.long()]), sub_k)
    assert np.array_equal(u16(vc[ids.long()]), sub_v)
