"""GPU parity of the fused append + decode (kvc_batch_decode_append_run,
PagedKVCache.append_and_decode): the cache bytes, the output and the lse
equal those of reshape_and_cache_flash followed by the decode run, bit for
bit, on the fused path and on the fallback (two calls) it takes when the
batch does not fit the fused kernel."""
import numpy as np
import pytest
import torch

from gpu_offloading_amd import workloads
from helpers import assert_attn_close, u16
from oracle import kv_oracle as orc

pytestmark = pytest.mark.gpu


def _two_caches(gpu, lens, hkv, hq, total, seed):
    from gpu_offloading_amd.kv_cache import PagedKVCache

    caches = []
    for _ in range(2):
        c = PagedKVCache(1, hkv, 128, max_seqs=len(lens), max_seq_len=max(lens) + 32,
                         num_qo_heads=hq, kv_page_budget=total,
                         free_page_order=workloads.randperm(total, seed), device=gpu,
                         workspace_bytes=1 << 24, staging_bytes=1 << 20)
        for s, n in enumerate(lens):
            c.ensure_pages(s, (n + 1 + 15) // 16)
        c.advance(list(range(len(lens))), lens)
        c.fill_kv_random(1.0, generator=torch.Generator(device=gpu).manual_seed(seed + 1))
        caches.append(c)
    return caches


def _step_both_ways(gpu, lens, hkv, hq, total, seed, order=None):
    a, b = _two_caches(gpu, lens, hkv, hq, total, seed)
    seqs = list(order) if order is not None else list(range(len(lens)))
    g = torch.Generator(device=gpu).manual_seed(seed + 2)
    n = len(seqs)
    k = torch.randn(n, hkv, 128, generator=g, device=gpu).to(torch.bfloat16)
    v = torch.randn(n, hkv, 128, generator=g, device=gpu).to(torch.bfloat16)
    q = torch.randn(n, hq, 128, generator=g, device=gpu).to(torch.bfloat16)
    slots = a.prepare_decode_step(seqs)
    a.append(0, k, v, slots)
    out_a, lse_a = a.decode(0, q, return_lse=True)
    b.prepare_decode_step(seqs)
    fused = b._decode_wrapper.fused_append_supported
    out_b, lse_b = b.append_and_decode(0, k, v, q, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(a.k_cache[0], b.k_cache[0]) and torch.equal(a.v_cache[0], b.v_cache[0])
    assert torch.equal(out_a, out_b) and torch.equal(lse_a, lse_b)
    # and the result is the attention over the appended token (oracle)
    lens_after = [int(b._seq_lens_cpu[s]) for s in seqs]
    indptr, lpl = orc.plan_decode(lens_after)
    idx = orc.page_indices(b.block_table.cpu().numpy(), seqs, indptr)
    ref, _ = orc.paged_decode(u16(q), u16(b.k_cache[0]), u16(b.v_cache[0]), indptr, idx, lpl)
    assert_attn_close(out_b.float().cpu().numpy(), ref)
    last = [int(idx[indptr[i + 1] - 1]) * 16 + int(lpl[i]) - 1 for i in range(n)]
    flat_k = u16(b.k_cache[0]).reshape(-1, hkv, 128)
    assert np.array_equal(flat_k[last], u16(k))
    return fused


def test_fused_append_matches_two_calls(gpu):
    """Mixtral shape (Hkv 8, G 4): contexts ending on every page offset,
    a one-token request, contexts across many segments; fused path taken."""
    rng = np.random.default_rng(90)
    lens = [0, 15, 16, 31, 1] + rng.integers(40, 900, 27).tolist()
    assert _step_both_ways(gpu, lens, 8, 32, 1200, 91)


def test_fused_append_step_order_and_mha(gpu):
    """Steps whose seq order differs from the slot order; MHA (Hkv 16, G 1)."""
    rng = np.random.default_rng(92)
    lens = rng.integers(1, 600, 20).tolist()
    order = rng.permutation(20).tolist()
    assert _step_both_ways(gpu, lens, 16, 16, 900, 93, order=order)


@pytest.mark.parametrize("hkv,hq,lens", [
    (8, 32, [128]),                     # the reference's batch-1 decode shape
    (8, 32, [0, 128, 33, 5, 255]),      # empty request, page ends, 16 pages after the step
    (16, 16, [40, 200]),                # MHA
    (4, 32, [100, 7]),                  # group 8
])
def test_fused_append_small_batch(gpu, hkv, hq, lens):
    """Small-batch schedules take the fused path too (one launch per layer)."""
    from gpu_offloading_amd.kv_cache import PagedKVCache  # noqa: F401

    total = sum((n + 1 + 15) // 16 for n in lens) + 8
    assert _step_both_ways(gpu, lens, hkv, hq, total, 96)


@pytest.mark.parametrize("hkv,hq,lens,total", [
    (8, 32, [3] * 1500, 1600),          # ~6 request ends per segment: append_pieces > 4
    (2, 8, [100, 7, 600, 64], 100),     # 2 KV heads, a 38-page request: one head per workgroup
])
def test_fused_append_falls_back_to_two_calls(gpu, hkv, hq, lens, total):
    assert not _step_both_ways(gpu, lens, hkv, hq, total, 94)


def test_fused_append_needs_a_step(gpu):
    from gpu_offloading_amd.kv_cache import PagedKVCache

    c = PagedKVCache(1, 8, 128, max_seqs=2, max_seq_len=64, num_qo_heads=32,
                     kv_page_budget=8, device=gpu, workspace_bytes=1 << 20,
                     staging_bytes=1 << 20)
    x = torch.zeros(2, 8, 128, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="prepare_decode_step"):
        c.append_and_decode(0, x, x, torch.zeros(2, 32, 128, dtype=torch.bfloat16, device=gpu))
