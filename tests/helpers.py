"""Small test helpers: bf16 <-> numpy bit patterns and seeded inputs."""
from __future__ import annotations

import numpy as np
import torch


def u16(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> numpy uint16 bit patterns."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_u16(a: np.ndarray, device=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
    return t.to(device) if device is not None else t


def randn_bf16(shape, seed, std=1.0, device=None):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(*shape, generator=g) * std).to(torch.bfloat16)
    return x.to(device) if device is not None else x


def oracle_decode_rows(q: np.ndarray, k_rows, v_rows, page_size: int = 16):
    """The oracle's paged decode of requests given as contiguous rows: request
    b's K/V rows ``k_rows[b]`` / ``v_rows[b]`` (uint16 bits ``[n_b, Hkv, D]``)
    are laid out in consecutive pages of a scratch cache, then
    ``orc.paged_decode`` attends ``q`` (bits ``[B, Hq, D]``) over them.
    Returns (out, lse)."""
    from oracle import kv_oracle as orc

    lens = [len(k) for k in k_rows]
    hkv, d = k_rows[0].shape[1:]
    indptr, lpl = orc.plan_decode(lens, page_size)
    total = max(int(indptr[-1]), 1)
    kc = np.zeros((total, page_size, hkv, d), np.uint16)
    vc = np.zeros_like(kc)
    for b, (k, v) in enumerate(zip(k_rows, v_rows)):
        flat_k = kc[indptr[b]:indptr[b + 1]].reshape(-1, hkv, d)
        flat_v = vc[indptr[b]:indptr[b + 1]].reshape(-1, hkv, d)
        flat_k[:len(k)] = k
        flat_v[:len(v)] = v
    indices = np.arange(int(indptr[-1]), dtype=np.int32)
    return orc.paged_decode(q, kc, vc, indptr, indices, lpl)


def assert_attn_close(got: np.ndarray, ref: np.ndarray, max_tol=2e-2, mean_tol=2e-3):
    """The decode-attention bar: max-abs-error <= 2e-2 and mean-abs-error
    <= 2e-3 of the bf16 output against an fp32 reference."""
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert np.isfinite(got).all(), "non-finite output"
    assert err.max() <= max_tol, f"max abs err {err.max():.3e} > {max_tol}"
    assert err.mean() <= mean_tol, f"mean abs err {err.mean():.3e} > {mean_tol}"
    return float(err.max()), float(err.mean())
