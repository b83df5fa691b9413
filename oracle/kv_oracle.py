"""CPU restatement (numpy) of the reference's paged KV-cache path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  Never part of the product path.

The reference engine (aojsd/GPU_Offloading, src/MoE/moe_engine.py) delegates the
arithmetic of this path to vLLM v0.17.1 (reshape_and_cache_flash, Triton slot
mapping / page-index kernels) and FlashInfer (BatchDecodeWithPagedKVCache),
which are not vendored in the reference and are absent here.  Each function
below restates the algorithm as the engine's call sites define it; the
citation is the file:line it follows.  How each function is pinned (checks
that do not retype its formula) is listed in tests/test_oracle.py.

bf16 tensors are numpy ``uint16`` bit patterns; arithmetic is float32 unless
stated.  Caches are ``[num_blocks, block_size, num_kv_heads, head_dim]``.
"""
from __future__ import annotations

from collections import deque
from typing import Optional, Sequence

import numpy as np

# --------------------------------------------------------------------- bf16


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32 (exact: bf16 is the top half)."""
    return (np.asarray(x, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round-to-nearest-even (NaN -> quiet NaN)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


# ------------------------------------------------------------- page pool


class FifoPagePool:
    """The engine's dynamic page pool (moe_engine.py:578-582, 4231-4297) and its
    CPU twin MockPageAllocator (src/MoE/scheduler.py:114-157): FIFO deque of page
    ids, popleft on alloc, extend on free, RuntimeError on exhaustion or on
    exceeding max_pages_per_seq, n <= 0 is a no-op.  The block table mirrors
    allocations (row entries = page ids, -1 when unallocated)."""

    def __init__(self, total_pages: int, max_seqs: int, max_pages_per_seq: int,
                 free_order: Optional[Sequence[int]] = None):
        self.total_pages = total_pages
        self.max_pages_per_seq = max_pages_per_seq
        self._init = list(range(total_pages)) if free_order is None else list(free_order)
        self.max_seqs = max_seqs
        self.reset()

    def reset(self):
        self.free = deque(self._init)
        self.pages = [[] for _ in range(self.max_seqs)]
        self.block_table = np.full((self.max_seqs, self.max_pages_per_seq), -1, dtype=np.int32)

    @property
    def pages_free(self):
        return len(self.free)

    @property
    def pages_in_use(self):
        return self.total_pages - len(self.free)

    def seq_pages(self, seq):
        return len(self.pages[seq])

    def alloc_pages(self, seq, n):
        if n <= 0:
            return
        cur = len(self.pages[seq])
        if cur + n > self.max_pages_per_seq:
            raise RuntimeError(f"Cannot allocate {n} pages for seq {seq}: would exceed "
                               f"max_pages_per_seq={self.max_pages_per_seq} (current={cur})")
        if len(self.free) < n:
            raise RuntimeError(f"Cannot allocate {n} pages for seq {seq}: only "
                               f"{len(self.free)} free pages remain (budget={self.total_pages})")
        new = [self.free.popleft() for _ in range(n)]
        self.pages[seq].extend(new)
        self.block_table[seq, cur:cur + n] = new

    def free_seq(self, seq):
        p = self.pages[seq]
        if not p:
            return
        self.free.extend(p)
        self.block_table[seq, :len(p)] = -1
        self.pages[seq] = []

    def ensure_pages(self, seq, needed):
        cur = len(self.pages[seq])
        if needed > cur:
            self.alloc_pages(seq, needed - cur)


# ---------------------------------------------------------- slot mapping


def slot_mapping(block_table: np.ndarray, seq_ids: Sequence[int], positions: Sequence[int],
                 page_size: int = 16) -> np.ndarray:
    """slot = block_table[seq, pos // page_size] * page_size + pos % page_size
    (moe_engine.py:1308-1316, 2677-2695, 1678-1695), int64."""
    seq = np.asarray(seq_ids, dtype=np.int64)
    pos = np.asarray(positions, dtype=np.int64)
    return block_table[seq, pos // page_size].astype(np.int64) * page_size + pos % page_size


def step_slot_mapping(block_table: np.ndarray, seq_ids: Sequence[int],
                      num_new_tokens: Sequence[int], num_computed: np.ndarray,
                      graph_n: int, page_size: int = 16):
    """Tokens laid out request by request; request r's tokens sit at positions
    num_computed[seq] + i; slots padded with -1 (PAD) and positions with 0 up to
    graph_n (moe_engine.py:3475-3541: prepare_pos_seq_lens +
    _compute_slot_mappings_kernel with PAD_ID=-1)."""
    seqs, pos = [], []
    for s, n in zip(seq_ids, num_new_tokens):
        for i in range(n):
            seqs.append(s)
            pos.append(int(num_computed[s]) + i)
    slots = np.full(graph_n, -1, dtype=np.int64)
    positions = np.zeros(graph_n, dtype=np.int32)
    if seqs:
        slots[:len(seqs)] = slot_mapping(block_table, seqs, pos, page_size)
        positions[:len(seqs)] = pos
    return slots, positions


# ---------------------------------------------------------------- plan


def plan_decode(seq_lens: Sequence[int], page_size: int = 16):
    """indptr = [0, cumsum(ceil(len / ps))]; last_page_len = len % ps, or ps when
    len is a non-zero multiple of ps (moe_engine.py:1907-1922)."""
    lens = np.asarray(seq_lens, dtype=np.int32)
    nblk = (lens + page_size - 1) // page_size
    indptr = np.zeros(len(lens) + 1, dtype=np.int32)
    np.cumsum(nblk, out=indptr[1:])
    lpl = lens % page_size
    lpl = np.where((lpl == 0) & (lens != 0), page_size, lpl).astype(np.int32)
    return indptr, lpl


def page_indices(block_table: np.ndarray, seq_ids: Sequence[int], indptr: np.ndarray) -> np.ndarray:
    """indices[indptr[r]:indptr[r+1]] = block_table[seq_ids[r], :n_r]
    (row index_select + _copy_page_indices_kernel, moe_engine.py:1937-1946)."""
    out = np.zeros(int(indptr[-1]), dtype=np.int32)
    for r, s in enumerate(seq_ids):
        n = indptr[r + 1] - indptr[r]
        out[indptr[r]:indptr[r + 1]] = block_table[s, :n]
    return out


# -------------------------------------------------------------- append


def reshape_and_cache(key: np.ndarray, value: np.ndarray, k_cache: np.ndarray,
                      v_cache: np.ndarray, slots: np.ndarray) -> None:
    """In place: cache.view(-1, H, D)[slot[i]] = src[i] for slot >= 0
    (reshape_and_cache_flash as called at moe_engine.py:2059-2062, "auto" dtype
    = plain copy; PyTorch twin :2196-2198 routes slot < 0 to a scratch row).
    Only the first len(slots) rows of key/value are used."""
    n = len(slots)
    nb, bs, h, d = k_cache.shape
    flat_k = k_cache.reshape(nb * bs, h, d)
    flat_v = v_cache.reshape(nb * bs, h, d)
    s = np.asarray(slots, dtype=np.int64)
    ok = (s >= 0) & (s < nb * bs)
    flat_k[s[ok]] = key[:n][ok]
    flat_v[s[ok]] = value[:n][ok]


# -------------------------------------------------------------- gather


def gather_kv(k_cache: np.ndarray, v_cache: np.ndarray, block_table: np.ndarray,
              seq_lens: Sequence[int], seq_starts: Optional[Sequence[int]] = None):
    """Contiguous KV of sequence rows 0..B-1: cache[bt[b, :nb]].flatten(0,1)
    [start:start+len] concatenated over b (the closed-form inverse of the append;
    cf. the un-permute in src/dense/scratch_examples/vllm_paged_attn.py:161-190)."""
    nb, bs, h, d = k_cache.shape
    ks, vs = [], []
    for b, ln in enumerate(seq_lens):
        st = 0 if seq_starts is None else int(seq_starts[b])
        pos = np.arange(st, st + ln)
        blk = block_table[b, pos // bs]
        ks.append(k_cache[blk, pos % bs])
        vs.append(v_cache[blk, pos % bs])
    if not ks:
        return np.zeros((0, h, d), k_cache.dtype), np.zeros((0, h, d), v_cache.dtype)
    return np.concatenate(ks), np.concatenate(vs)


# ----------------------------------------------------- decode attention


def _request_kv(k_cache: np.ndarray, v_cache: np.ndarray, pages: np.ndarray, n: int):
    """K and V (float32 ``[n, Hkv, D]``) of a request's first ``n`` tokens on
    ``pages``, and which of them are present.  A page id outside
    ``[0, num_blocks)`` (-1 for an unallocated block-table entry) is a missing
    page: its tokens are hidden from the attention (their K/V rows read as 0
    and they are masked out), the error behaviour this build's kernels define
    for a corrupt page list (the engine never plans one; FlashInfer would read
    out of bounds)."""
    nb, ps = k_cache.shape[:2]
    pages = np.asarray(pages, np.int64)
    ok = (pages >= 0) & (pages < nb)
    safe = np.where(ok, pages, 0)
    present = np.repeat(ok, ps)[:n]
    K = bf16_to_f32(k_cache[safe].reshape(-1, *k_cache.shape[2:])[:n])
    V = bf16_to_f32(v_cache[safe].reshape(-1, *v_cache.shape[2:])[:n])
    K[~present] = 0.0
    V[~present] = 0.0
    return K, V, present


def paged_decode(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                 indptr: np.ndarray, indices: np.ndarray, last_page_len: np.ndarray,
                 sm_scale: Optional[float] = None):
    """fp32 naive paged GQA decode attention, the semantics of FlashInfer
    BatchDecodeWithPagedKVCacheWrapper.run as the engine calls it
    (moe_engine.py:3907-3909; plan :1949-1955 with pos_encoding_mode "NONE",
    default sm_scale 1/sqrt(head_dim)):
        out[b, h] = softmax(sm_scale * q[b, h] . K_b^T) . V_b,  kv head = h // (Hq/Hkv)
    over the len_b = (pages-1)*ps + last_page_len[b] tokens of request b.
    Tokens of missing pages (``_request_kv``) are hidden.
    q: bf16 bits [B, Hq, D]; returns (out float32 [B, Hq, D], lse float32 [B, Hq],
    natural log; a request with no (present) token gives out 0, lse -inf)."""
    q = bf16_to_f32(q)
    B, Hq, D = q.shape
    nb, ps, Hkv, _ = k_cache.shape
    G = Hq // Hkv
    scale = np.float32(1.0 / np.sqrt(D) if sm_scale is None else sm_scale)
    out = np.zeros((B, Hq, D), np.float32)
    lse = np.full((B, Hq), -np.inf, np.float32)
    for b in range(B):
        pages = indices[indptr[b]:indptr[b + 1]]
        if len(pages) == 0:
            continue
        n = (len(pages) - 1) * ps + int(last_page_len[b])
        K, V, present = _request_kv(k_cache, v_cache, pages, n)
        if not present.any():
            continue
        for h in range(Hkv):
            qg = q[b, h * G:(h + 1) * G]                      # [G, D]
            s = (qg @ K[:, h, :].T) * scale                  # [G, n]
            s = np.where(present[None, :], s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            p = np.exp(s - m)
            l = p.sum(axis=1, keepdims=True)
            out[b, h * G:(h + 1) * G] = (p @ V[:, h, :]) / l
            lse[b, h * G:(h + 1) * G] = (m + np.log(l))[:, 0]
    return out, lse


def paged_prefill(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                  qo_indptr: np.ndarray, kv_indptr: np.ndarray, indices: np.ndarray,
                  last_page_len: np.ndarray, causal: bool = True,
                  sm_scale: Optional[float] = None):
    """fp32 naive paged prefill attention, the semantics of FlashInfer
    BatchPrefillWithPagedKVCacheWrapper.run as the engine calls it for
    continuation prefills (moe_engine.py:3939-3941; plan :3710-3727 with
    causal=True, pos_encoding_mode "NONE", default sm_scale 1/sqrt(head_dim)).
    Request b owns query rows qo_indptr[b]..qo_indptr[b+1] (q_len) and the
    kv_len = (pages-1)*ps + last_page_len[b] cached tokens of its pages; with
    causal masking query i sees keys j <= i + kv_len - q_len (the chunk is
    the tail of the cache); tokens of missing pages (``_request_kv``) are
    hidden.  A query that sees nothing gives out 0, lse -inf.
    q: bf16 bits [total_q, Hq, D]; returns (out float32, lse float32 natural log)."""
    q = bf16_to_f32(q)
    T, Hq, D = q.shape
    nb, ps, Hkv, _ = k_cache.shape
    G = Hq // Hkv
    scale = np.float32(1.0 / np.sqrt(D) if sm_scale is None else sm_scale)
    out = np.zeros((T, Hq, D), np.float32)
    lse = np.full((T, Hq), -np.inf, np.float32)
    for b in range(len(qo_indptr) - 1):
        q0, q1 = int(qo_indptr[b]), int(qo_indptr[b + 1])
        pages = indices[kv_indptr[b]:kv_indptr[b + 1]]
        if q1 == q0 or len(pages) == 0:
            continue
        q_len = q1 - q0
        n = (len(pages) - 1) * ps + int(last_page_len[b])
        K, V, present = _request_kv(k_cache, v_cache, pages, n)
        seen = np.ones((q_len, n), bool)
        if causal:
            seen = np.arange(n)[None, :] <= np.arange(q_len)[:, None] + (n - q_len)
        seen &= present[None, :]
        any_seen = seen.any(axis=1)
        for h in range(Hkv):
            for g in range(G):
                hq = h * G + g
                s = (q[q0:q1, hq] @ K[:, h, :].T) * scale           # [q_len, n]
                s = np.where(seen, s, -np.inf)
                m = np.where(any_seen, s.max(axis=1), 0.0)[:, None]
                p = np.where(seen, np.exp(s - m), 0.0)
                l = p.sum(axis=1, keepdims=True)
                with np.errstate(invalid="ignore", divide="ignore"):
                    o = np.where(l > 0, (p @ V[:, h, :]) / np.where(l > 0, l, 1.0), 0.0)
                    lse[q0:q1, hq] = np.where(any_seen, (m + np.log(np.where(l > 0, l, 1.0)))[:, 0],
                                              -np.inf)
                out[q0:q1, hq] = o
    return out, lse


def merge_attention_states(out1, lse1, out2, lse2):
    """src/dense/offload_kv_attn.py:24-39 in fp32: lse = logaddexp(lse1, lse2),
    out = out1 * exp(lse1 - lse) + out2 * exp(lse2 - lse)."""
    o1 = np.asarray(out1, np.float32)
    o2 = np.asarray(out2, np.float32)
    l1 = np.asarray(lse1, np.float32)[..., None]
    l2 = np.asarray(lse2, np.float32)[..., None]
    new = np.logaddexp(l1, l2)
    with np.errstate(invalid="ignore"):
        w1 = np.where(np.isneginf(new), 0.0, np.exp(l1 - new)).astype(np.float32)
        w2 = np.where(np.isneginf(new), 0.0, np.exp(l2 - new)).astype(np.float32)
    return o1 * w1 + o2 * w2, new[..., 0]


# ------------------------------------------------- x-packed layout (f3)


def elem_to_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    """2-byte element bits (uint16) to float32: "bf16" or "fp16"."""
    if dtype == "bf16":
        return bf16_to_f32(x)
    return np.asarray(x, np.uint16).view(np.float16).astype(np.float32)


def reshape_and_cache_xpacked(key: np.ndarray, value: np.ndarray, key_cache: np.ndarray,
                              value_cache: np.ndarray, slot_mapping: np.ndarray) -> None:
    """vLLM reshape_and_cache as called at src/dense/include/paged_transformer.py:290-294,
    in place on bits: key_cache [nb, H, D/x, bs, x], value_cache [nb, H, D, bs];
    token i with slot s >= 0 goes to block s // bs, offset s % bs."""
    nb, H, Dx, bs, x = key_cache.shape
    for i, s in enumerate(np.asarray(slot_mapping, np.int64)):
        if s < 0 or s >= nb * bs:
            continue
        blk, off = divmod(int(s), bs)
        key_cache[blk, :, :, off, :] = key[i].reshape(H, Dx, x)
        value_cache[blk, :, :, off] = value[i]


def xpacked_to_nhd(key_cache: np.ndarray, value_cache: np.ndarray):
    """The x-packed caches re-laid as the flat NHD layout [nb, bs, H, D]."""
    nb, H, Dx, bs, x = key_cache.shape
    k = key_cache.transpose(0, 3, 1, 2, 4).reshape(nb, bs, H, Dx * x)
    v = value_cache.transpose(0, 3, 1, 2)
    return np.ascontiguousarray(k), np.ascontiguousarray(v)


def paged_attention_xpacked(q: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray,
                            block_tables: np.ndarray, seq_lens: np.ndarray, scale: float,
                            dtype: str = "fp16", partition: int = 512):
    """vLLM paged_attention_v1/v2 over the x-packed layout
    (paged_transformer.py:325-332): out[b, h] = softmax(scale q.K^T) V over
    the seq_lens[b] tokens of block_tables[b], kv head = h // (H / Hkv), in
    fp32.  Also returns v2's per-partition scratch: max_logits[b, h, p] (max
    scaled logit of the 512-token partition), exp_sums[b, h, p] (sum of
    exp(logit - max)) and tmp_out[b, h, p] (the partition's normalised
    output), fp32.  q: element bits [B, H, D]."""
    qf = elem_to_f32(q, dtype)
    B, Hq, D = qf.shape
    kn, vn = xpacked_to_nhd(key_cache, value_cache)
    Kf = elem_to_f32(kn, dtype)
    Vf = elem_to_f32(vn, dtype)
    bs, Hkv = kn.shape[1], kn.shape[2]
    G = Hq // Hkv
    P = max(1, max((int(n) + partition - 1) // partition for n in seq_lens))
    out = np.zeros((B, Hq, D), np.float32)
    ml = np.full((B, Hq, P), -np.inf, np.float32)
    es = np.zeros((B, Hq, P), np.float32)
    tmp = np.zeros((B, Hq, P, D), np.float32)
    for b in range(B):
        n = int(seq_lens[b])
        if n == 0:
            continue
        pages = block_tables[b, :(n + bs - 1) // bs]
        K = Kf[pages].reshape(-1, Hkv, D)[:n]
        V = Vf[pages].reshape(-1, Hkv, D)[:n]
        for h in range(Hq):
            s = (K[:, h // G] @ qf[b, h]) * np.float32(scale)
            e = np.exp(s - s.max())
            out[b, h] = (e @ V[:, h // G]) / e.sum()
            for p0 in range(0, n, partition):
                sp = s[p0:p0 + partition]
                ep = np.exp(sp - sp.max())
                ml[b, h, p0 // partition] = sp.max()
                es[b, h, p0 // partition] = ep.sum()
                tmp[b, h, p0 // partition] = (ep @ V[p0:p0 + partition, h // G]) / ep.sum()
    return out, ml, es, tmp


# ---------------------------------------------------------------- swap


def gather_blocks(k_cache: np.ndarray, v_cache: np.ndarray, block_ids: Sequence[int]) -> np.ndarray:
    """Staging image [n, 2, block_bytes] (K block then V block) of block_ids
    (index_select; the block-granular form of kv_snapshot, moe_engine.py:4163-4170)."""
    ids = np.asarray(block_ids, dtype=np.int64)
    kb = k_cache[ids].reshape(len(ids), -1).view(np.uint8)
    vb = v_cache[ids].reshape(len(ids), -1).view(np.uint8)
    return np.stack([kb, vb], axis=1)


def scatter_blocks(staging: np.ndarray, block_ids: Sequence[int], k_cache: np.ndarray,
                   v_cache: np.ndarray) -> None:
    """Inverse of gather_blocks (index_copy; block-granular kv_restore,
    moe_engine.py:4172-4183)."""
    ids = np.asarray(block_ids, dtype=np.int64)
    shp = k_cache.shape[1:]
    k_cache[ids] = staging[:, 0].copy().view(k_cache.dtype).reshape((len(ids),) + shp)
    v_cache[ids] = staging[:, 1].copy().view(v_cache.dtype).reshape((len(ids),) + shp)
