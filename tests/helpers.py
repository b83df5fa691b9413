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


def assert_attn_close(got: np.ndarray, ref: np.ndarray, max_tol=2e-2, mean_tol=2e-3):
    """The decode-attention bar: max-abs-error <= 2e-2 and mean-abs-error
    <= 2e-3 of the bf16 output against an fp32 reference."""
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert np.isfinite(got).all(), "non-finite output"
    assert err.max() <= max_tol, f"max abs err {err.max():.3e} > {max_tol}"
    assert err.mean() <= mean_tol, f"mean abs err {err.mean():.3e} > {mean_tol}"
    return float(err.max()), float(err.mean())
