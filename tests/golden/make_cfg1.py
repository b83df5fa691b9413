"""Write tests/golden/cfg1.npz: the configuration-1 fixture.

Configuration 1 of the benchmark set: 2 layers, Hkv=8, Hq=32, D=128, 16-token
pages, a 256-block pool whose free list is a seeded permutation, sequences of
37, 128, 255 and 513 tokens.  All inputs are drawn from seeded CPU
torch.Generator streams (reproducible from the seeds alone); the expected
outputs come from the CPU oracle (oracle/kv_oracle.py), which follows the
reference engine's semantics (no reference-produced vectors exist for this
path).  Stored: the block table and slot mapping after allocation, SHA-256 of
every appended cache and of the gathered K/V, and the fp32 decode output and
log-sum-exp of one decode step per layer (each sequence appends one token,
then attends over len + 1 tokens).

Run from the repository root:  python tests/golden/make_cfg1.py
"""
import hashlib
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from gpu_offloading_amd import workloads  # noqa: E402
from oracle import kv_oracle as orc  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cfg1.npz")


def u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def inputs(layer, n, h, d, hq, b):
    """Seeded bf16 inputs of one layer: prompt K/V, the step's new K/V, q."""
    return (u16(workloads.randn_bf16((n, h, d), 1000 + 10 * layer)),
            u16(workloads.randn_bf16((n, h, d), 1001 + 10 * layer)),
            u16(workloads.randn_bf16((b, h, d), 1002 + 10 * layer)),
            u16(workloads.randn_bf16((b, h, d), 1003 + 10 * layer)),
            u16(workloads.randn_bf16((b, hq, d), 1004 + 10 * layer)))


def compute():
    cfg = workloads.config1(seed=0)
    sh = cfg.shape
    lens = cfg.seq_lens
    b = len(lens)
    pool = orc.FifoPagePool(cfg.total_pages, b, 64, free_order=cfg.free_order)
    for s, ln in enumerate(lens):
        pool.ensure_pages(s, (ln + 1 + 15) // 16)      # room for the decode token
    seqs = np.concatenate([[s] * ln for s, ln in enumerate(lens)])
    pos = np.concatenate([np.arange(ln) for ln in lens])
    slots = orc.slot_mapping(pool.block_table, seqs, pos)
    step_slots = orc.slot_mapping(pool.block_table, range(b), lens)
    lens1 = [ln + 1 for ln in lens]
    indptr, lpl = orc.plan_decode(lens1)
    indices = orc.page_indices(pool.block_table, range(b), indptr)
    out = {"block_table": pool.block_table, "slots": slots, "step_slots": step_slots,
           "indptr": indptr, "last_page_len": lpl, "indices": indices,
           "seq_lens": np.asarray(lens, np.int32)}
    n = len(slots)
    for layer in range(sh.num_layers):
        k, v, kn, vn, q = inputs(layer, n, sh.num_kv_heads, sh.head_dim, sh.num_qo_heads, b)
        kc = np.zeros((cfg.total_pages, 16, sh.num_kv_heads, sh.head_dim), np.uint16)
        vc = np.zeros_like(kc)
        orc.reshape_and_cache(k, v, kc, vc, slots)
        gk, gv = orc.gather_kv(kc, vc, pool.block_table, lens)
        orc.reshape_and_cache(kn, vn, kc, vc, step_slots)
        o, l = orc.paged_decode(q, kc, vc, indptr, indices, lpl)
        out[f"sha_kcache_{layer}"] = np.array(sha(kc))
        out[f"sha_vcache_{layer}"] = np.array(sha(vc))
        out[f"sha_gather_k_{layer}"] = np.array(sha(gk))
        out[f"sha_gather_v_{layer}"] = np.array(sha(gv))
        out[f"decode_out_{layer}"] = o
        out[f"decode_lse_{layer}"] = l
    return out


if __name__ == "__main__":
    np.savez_compressed(OUT, **compute())
    print("wrote", OUT, os.path.getsize(OUT), "bytes")
