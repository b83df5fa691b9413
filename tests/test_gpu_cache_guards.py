"""GPU checks of the cache manager's guards: planning calls refuse bad
sequence ids and oversized sequences before anything is launched, the gather
and page-index kernels never write past the outputs they are given (their own
bounds checks, on device metadata larger than the buffers), and a sequence
freed while its restore is still in flight hands its pages to the next owner
only after the restore wrote them."""
import numpy as np
import pytest
import torch

from gpu_offloading_amd import ops
from gpu_offloading_amd.kv_cache import PagedKVCache
from helpers import randn_bf16, u16

pytestmark = pytest.mark.gpu


def _cache(gpu, layers=1, max_seqs=4, max_seq_len=256, budget=64, **kw):
    return PagedKVCache(layers, 8, 128, max_seqs=max_seqs, max_seq_len=max_seq_len,
                        num_qo_heads=32, kv_page_budget=budget, device=gpu,
                        workspace_bytes=kw.pop("workspace_bytes", 1 << 22),
                        staging_bytes=kw.pop("staging_bytes", 1 << 20), **kw)


def test_planning_misuse_raises(gpu):
    print("guards: planning misuse", flush=True)
    cache = _cache(gpu)
    cache.ensure_pages(0, 2)
    cache.advance([0], [20])
    for bad in ([-1], [0, 0], [4]):
        with pytest.raises(ValueError, match="distinct"):
            cache.plan_decode(bad)
        with pytest.raises(ValueError, match="distinct"):
            cache.plan_prefill(bad, [0] * len(bad))
        with pytest.raises(ValueError, match="distinct"):
            cache.gather(0, bad)
        with pytest.raises(ValueError, match="distinct"):
            cache.prepare_decode_step(bad)
    short = torch.empty(19, 8, 128, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(RuntimeError, match="rows"):
        cache.gather(0, [0], out_key=short)
    with pytest.raises(RuntimeError, match="rows"):
        cache.gather(0, [0], out_value=short)
    cache.advance([1], [300])                   # past max_seq_len: refused, not truncated
    with pytest.raises(RuntimeError, match="max_seq_len"):
        cache.plan_decode([1])
    with pytest.raises(RuntimeError, match="max_seq_len"):
        cache.plan_prefill([1], [1])
    # the good calls still work afterwards
    cache.plan_decode([0])
    k, v = cache.gather(0, [0])
    torch.cuda.synchronize()
    assert k.shape == (20, 8, 128)


def test_gather_and_page_indices_stay_inside_their_outputs(gpu):
    """Device metadata that claims more rows than the output holds: the
    kernels write only inside the output (the rest of the surrounding buffer
    keeps its sentinel) and count the rows they skipped."""
    print("guards: kernel output bounds", flush=True)
    kc = randn_bf16((8, 16, 8, 128), 1, device=gpu)
    vc = randn_bf16((8, 16, 8, 128), 2, device=gpu)
    bt = torch.arange(8, dtype=torch.int32, device=gpu).view(1, 8)
    big_k = torch.full((128, 8, 128), 7.0, dtype=torch.bfloat16, device=gpu)
    big_v = torch.full((128, 8, 128), 7.0, dtype=torch.bfloat16, device=gpu)
    cu = torch.tensor([0, 100], dtype=torch.int32, device=gpu)   # 100 rows claimed
    oob = torch.zeros(1, dtype=torch.int32, device=gpu)
    ops.gather_kv(kc, vc, bt, cu, 100, big_k[:60], big_v[:60], oob_count=oob)
    torch.cuda.synchronize()
    assert int(oob.item()) == 40
    flat_k = kc.view(-1, 8, 128)
    assert torch.equal(big_k[:60], flat_k[:60]) and torch.equal(big_v[:60], vc.view(-1, 8, 128)[:60])
    assert (big_k[60:] == 7.0).all() and (big_v[60:] == 7.0).all()

    table = torch.arange(4 * 16, dtype=torch.int32, device=gpu).view(4, 16)
    indptr = torch.tensor([0, 16, 32, 48], dtype=torch.int32, device=gpu)
    buf = torch.full((64,), -5, dtype=torch.int32, device=gpu)
    ops.copy_page_indices(table, indptr, buf[:40])              # 48 entries claimed
    torch.cuda.synchronize()
    assert buf[:40].tolist() == list(range(32)) + list(range(32, 40))
    assert (buf[40:] == -5).all()


def test_free_during_restore_orders_the_pages_next_owner(gpu):
    """Sequence 0 is swapped out, restored, and freed while the restore may
    still run; its pages go to sequence 1, whose K/V are appended on the
    current stream right away.  Every page must end up holding sequence 1's
    rows (the append ordered after the restore's scatter)."""
    print("guards: free during restore", flush=True)
    layers, pages = 4, 128
    cache = _cache(gpu, layers=layers, max_seqs=2, max_seq_len=pages * 16, budget=pages,
                   staging_bytes=1 << 24)
    n = pages * 16
    cache.ensure_pages(0, pages)
    cache.advance([0], [n])
    cache.fill_kv_random(1.0, generator=torch.Generator(device=gpu).manual_seed(3))
    torch.cuda.synchronize()
    handle = cache.swap_out([0])
    cache.swap_in(handle)          # 4 layers x 128 blocks x 64 KB through a 16 MB staging
    cache.free_seq(0)              # the restore may still be writing these pages
    cache.ensure_pages(1, pages)   # the same pages, now sequence 1's
    slots = cache.slot_mapping([1], [n])
    ks = [randn_bf16((n, 8, 128), 10 + layer, device=gpu) for layer in range(layers)]
    vs = [randn_bf16((n, 8, 128), 20 + layer, device=gpu) for layer in range(layers)]
    for layer in range(layers):
        cache.append(layer, ks[layer], vs[layer], slots)
    cache.advance([1], [n])
    for layer in range(layers):
        gk, gv = cache.gather(layer, [1])
        torch.cuda.synchronize()
        assert np.array_equal(u16(gk), u16(ks[layer])), f"layer {layer}: K overwritten"
        assert np.array_equal(u16(gv), u16(vs[layer])), f"layer {layer}: V overwritten"
    cache.synchronize_swaps()
