"""torch-CPU restatement of the oracle's paged KV-cache functions, for timing
the reference semantics on all of a host's cores.

TEST INFRASTRUCTURE ONLY: imported by tests/ and by the cpu_baseline leg of
bench.py, never part of the product path.  Each function computes what the
numpy oracle (oracle/kv_oracle.py) computes for the same inputs -- bit for bit
for the byte work, within float32 rounding for attention -- with torch's
multi-threaded CPU kernels (index_copy_, index_select, batched matmul):

* append  = ``reshape_and_cache``: index_copy_ into cache.view(-1, Hkv, D),
  slots < 0 skipped (reshape_and_cache_flash as called at
  src/MoE/moe_engine.py:2059-2062; PyTorch twin :2196-2198);
* gather  = ``gather_kv``: index_select of each sequence's block-table rows
  (closed form cache[bt[seq, :nb]].flatten(0, 1)[:len]);
* decode  = ``paged_decode``: fp32 naive softmax(q K^T / sqrt(D)) V with
  kv head = q head // (Hq / Hkv), per request (FlashInfer decode as called at
  moe_engine.py:3907-3909);
* swap    = ``gather_blocks`` / ``scatter_blocks``: row indexing of whole
  blocks into a host staging image and index_copy_ back (the block-granular
  kv_snapshot / kv_restore, moe_engine.py:4163-4183).

bf16 tensors are torch.bfloat16 here (the oracle uses uint16 bit patterns of
the same values).
"""
from __future__ import annotations

import math
from typing import Optional, Sequence

import torch


def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                      v_cache: torch.Tensor, slots: torch.Tensor) -> None:
    """In place: cache.view(-1, H, D)[slot[i]] = src[i] for 0 <= slot < capacity."""
    nb, bs, h, d = k_cache.shape
    n = slots.numel()
    ok = (slots >= 0) & (slots < nb * bs)
    idx = slots[ok]
    k_cache.view(nb * bs, h, d).index_copy_(0, idx, key[:n][ok])
    v_cache.view(nb * bs, h, d).index_copy_(0, idx, value[:n][ok])


def gather_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
              seq_lens: Sequence[int]):
    """Contiguous [sum(len), H, D] K and V of block-table rows 0..B-1."""
    bs = k_cache.shape[1]
    ks, vs = [], []
    for b, ln in enumerate(seq_lens):
        pages = block_table[b, :(ln + bs - 1) // bs].long()
        ks.append(k_cache.index_select(0, pages).flatten(0, 1)[:ln])
        vs.append(v_cache.index_select(0, pages).flatten(0, 1)[:ln])
    return torch.cat(ks), torch.cat(vs)


def paged_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                 indptr: torch.Tensor, indices: torch.Tensor, last_page_len: torch.Tensor,
                 sm_scale: Optional[float] = None):
    """fp32 paged GQA decode; returns (out float32 [B, Hq, D], lse [B, Hq])."""
    B, Hq, D = q.shape
    _, ps, Hkv, _ = k_cache.shape
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if sm_scale is None else sm_scale
    out = torch.zeros(B, Hq, D, dtype=torch.float32)
    lse = torch.full((B, Hq), -math.inf, dtype=torch.float32)
    for b in range(B):
        p0, p1 = int(indptr[b]), int(indptr[b + 1])
        if p1 == p0:
            continue
        n = (p1 - p0 - 1) * ps + int(last_page_len[b])
        pages = indices[p0:p1].long()
        K = k_cache.index_select(0, pages).flatten(0, 1)[:n].float().permute(1, 2, 0)  # [Hkv, D, n]
        V = v_cache.index_select(0, pages).flatten(0, 1)[:n].float().transpose(0, 1)   # [Hkv, n, D]
        qg = q[b].float().view(Hkv, G, D)
        s = torch.bmm(qg, K) * scale                                                 # [Hkv, G, n]
        m = s.amax(dim=2, keepdim=True)
        p = torch.exp(s - m)
        l = p.sum(dim=2, keepdim=True)
        out[b] = (torch.bmm(p, V) / l).reshape(Hq, D)
        lse[b] = (m + torch.log(l)).reshape(Hq)
    return out, lse


def gather_blocks(k_cache: torch.Tensor, v_cache: torch.Tensor,
                  block_ids: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Staging image [n, 2, block_bytes] (uint8) of the blocks, K then V."""
    ids = block_ids.long()
    nb = k_cache.shape[0]
    kb = k_cache.reshape(nb, -1)[ids].view(torch.uint8)
    vb = v_cache.reshape(nb, -1)[ids].view(torch.uint8)
    if out is None:
        return torch.stack([kb, vb], dim=1)
    out[:, 0].copy_(kb)
    out[:, 1].copy_(vb)
    return out


def scatter_blocks(staging: torch.Tensor, block_ids: torch.Tensor, k_cache: torch.Tensor,
                   v_cache: torch.Tensor) -> None:
    """Inverse of gather_blocks (index_copy_ of whole blocks)."""
    ids = block_ids.long()
    shp = (ids.numel(),) + tuple(k_cache.shape[1:])
    k_cache.index_copy_(0, ids, staging[:, 0].contiguous().view(k_cache.dtype).view(shp))
    v_cache.index_copy_(0, ids, staging[:, 1].contiguous().view(v_cache.dtype).view(shp))
