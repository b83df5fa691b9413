"""Host-side layout of the layer-wise KV offload (CPU): block counts,
scratchpad placement and block tables follow the dense sandbox's rules
(src/dense/include/paged_offload_transformer.py:55-230)."""
import math

import pytest
import torch

from gpu_offloading_amd.offload import PagedOffloadKV


@pytest.mark.parametrize("ratio,mode", [(0.5, "random"), (0.25, "contiguous"), (0.0, "random")])
def test_offload_layout(ratio, mode):
    dec, pre, L = [100, 37, 300, 15], [40, 17], 4
    kv = PagedOffloadKV(dec, pre, L, 2, 128, ratio, device="cpu", allocation_mode=mode, seed=1)
    blocks = [math.ceil(n / 16) for n in pre] + [math.ceil((n + 1) / 16) for n in dec]
    assert kv.blocks_per_seq == blocks
    assert kv.offload_counts == [int(b * ratio) for b in blocks]
    P = len(pre)
    assert kv.prefill_offload_blocks == sum(kv.offload_counts[:P])
    assert kv.decode_offload_blocks == sum(kv.offload_counts[P:])
    off = kv.offload_blocks
    res_pool = sum(blocks) + sum(b - o for b, o in zip(blocks, kv.offload_counts)) * (L - 1)
    assert kv.heap_blocks == res_pool + 2 * off
    assert kv.scratchpad_ranges == [(res_pool, res_pool + off), (res_pool + off, res_pool + 2 * off)]
    bt = kv.block_tables_cpu
    resident = []
    for b, n_tot in enumerate(blocks):
        resident += bt[0, b, :n_tot].tolist()
        for layer in range(1, L):
            n_off = kv.offload_counts[b]
            sp = kv.scratchpad_ranges[layer % 2][0] + kv.scratchpad_seq_offsets[b]
            assert bt[layer, b, :n_off].tolist() == list(range(sp, sp + n_off))
            resident += bt[layer, b, n_off:n_tot].tolist()
    # every resident block is used once, all inside the resident pool
    assert sorted(resident) == list(range(res_pool))
    # decode sequences first inside a scratchpad, then prefill sequences
    offs = kv.scratchpad_seq_offsets
    assert offs[P] == 0 and (P == 0 or offs[0] == kv.decode_offload_blocks)
    # slot mapping: prefill tokens in order, then each decode's new token
    sm = kv.slot_mapping
    assert sm.shape == (L, sum(pre) + len(dec))
    for layer in range(L):
        t = sum(pre) + 2                      # decode sequence 2, position 300
        b, pos = P + 2, dec[2]
        assert int(sm[layer, t]) == int(bt[layer, b, pos // 16]) * 16 + pos % 16
        assert int(sm[layer, 41]) == int(bt[layer, 1, 1 // 16]) * 16 + 1   # prefill 1, token 1
    assert kv.decode_context_lens.tolist() == [n + 1 for n in dec]


def test_offload_history_lands_in_host_buffers_and_heap():
    kv = PagedOffloadKV([40], [], 2, 2, 128, 0.5, device="cpu")
    k = torch.arange(40 * 2 * 128, dtype=torch.float32).view(40, 2, 128).half()
    v = -k
    kv.load_history(1, 0, k, v)
    n_off = kv.offload_counts[0]                       # int(3 * 0.5) = 1 block offloaded
    assert n_off == 1
    # token 5, head 1, dim 37 of the offloaded block is in the host buffer
    x = kv.x
    assert kv.k_offload_cpu[0][0, 1, 37 // x, 5, 37 % x] == k[5, 1, 37]
    assert kv.v_offload_cpu[0][0, 1, 37, 5] == v[5, 1, 37]
    # token 20 (block 1) is resident in the heap at the table's id
    blk = int(kv.block_tables_cpu[1, 0, 1])
    assert kv.key_heap[blk, 0, 3, 4, 2] == k[20, 0, 3 * x + 2]
    assert kv.val_heap[blk, 1, 100, 4] == v[20, 1, 100]
