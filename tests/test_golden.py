"""The committed configuration-1 fixture (tests/golden/cfg1.npz, written by
tests/golden/make_cfg1.py from seeded inputs and the CPU oracle).

CPU: the oracle still reproduces the fixture (guards the checker itself).
GPU: the HIP path, driven through PagedKVCache like the engine drives it
(allocate, append the prompt, gather, one decode step), matches the fixture:
block table and slots exactly, cache and gather SHA-256 bit-exact, decode
within max 2e-2 / mean 2e-3."""

import numpy as np
import pytest
import torch

from golden.make_cfg1 import OUT, compute, inputs, sha
from helpers import assert_attn_close, from_u16, u16

FIX = np.load(OUT, allow_pickle=False)


def test_oracle_reproduces_the_fixture():
    got = compute()
    assert sorted(got) == sorted(FIX.files)
    for k in FIX.files:
        if k.startswith("decode_"):
            np.testing.assert_allclose(got[k], FIX[k], rtol=1e-5, atol=1e-6)
        else:
            assert np.array_equal(got[k], FIX[k]), k


@pytest.mark.gpu
def test_hip_path_matches_the_fixture(gpu):
    from gpu_offloading_amd import workloads
    from gpu_offloading_amd.kv_cache import PagedKVCache

    cfg = workloads.config1(seed=0)
    sh = cfg.shape
    lens = cfg.seq_lens
    b = len(lens)
    cache = PagedKVCache(sh.num_layers, sh.num_kv_heads, sh.head_dim, max_seqs=b,
                         max_seq_len=64 * 16, num_qo_heads=sh.num_qo_heads,
                         kv_page_budget=cfg.total_pages, free_page_order=cfg.free_order,
                         device=gpu)
    seqs = list(range(b))
    for s, ln in enumerate(lens):
        cache.ensure_pages(s, (ln + 1 + 15) // 16)
    assert np.array_equal(cache.block_table.cpu().numpy(), FIX["block_table"])
    slots = cache.slot_mapping(seqs, lens)
    assert np.array_equal(slots.cpu().numpy(), FIX["slots"])
    n = len(FIX["slots"])
    prompt = [inputs(layer, n, sh.num_kv_heads, sh.head_dim, sh.num_qo_heads, b)
              for layer in range(sh.num_layers)]
    for layer, (k, v, _, _, _) in enumerate(prompt):
        cache.append(layer, from_u16(k, gpu), from_u16(v, gpu), slots)
    cache.advance(seqs, lens)
    for layer in range(sh.num_layers):
        gk, gv = cache.gather(layer, seqs)
        assert sha(u16(gk)) == str(FIX[f"sha_gather_k_{layer}"])
        assert sha(u16(gv)) == str(FIX[f"sha_gather_v_{layer}"])
    step_slots = cache.prepare_decode_step(seqs)
    assert np.array_equal(step_slots.cpu().numpy(), FIX["step_slots"])
    for layer, (_, _, kn, vn, q) in enumerate(prompt):
        cache.append(layer, from_u16(kn, gpu), from_u16(vn, gpu), step_slots)
        out, lse = cache.decode(layer, from_u16(q, gpu), return_lse=True)
        torch.cuda.synchronize()
        assert sha(u16(cache.k_cache[layer])) == str(FIX[f"sha_kcache_{layer}"])
        assert sha(u16(cache.v_cache[layer])) == str(FIX[f"sha_vcache_{layer}"])
        assert_attn_close(out.float().cpu().numpy(), FIX[f"decode_out_{layer}"])
        assert np.allclose(lse.cpu().numpy(), FIX[f"decode_lse_{layer}"], atol=1e-3, rtol=1e-4)
