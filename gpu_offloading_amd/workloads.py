"""Seeded synthetic workloads of the benchmark configurations and their
algorithmic byte counts.

Inputs are drawn with a CPU ``torch.Generator`` (so the same seed gives the
same bf16 values on any box with this torch build) and are moved to the GPU
afterwards; large benchmark fills may be drawn on the device instead.

Configurations (the KV layout is always 16-token pages, bf16, head_dim 128):
  1  small case: 2 layers, Hkv 8 / Hq 32, pool of 256 blocks with a shuffled
     free list, four sequences of 37, 128, 255 and 513 tokens
  2  Mixtral-shaped decode step: 32 layers, Hkv 8 / Hq 32, batch 64, context
     uniform in [512, 4096], blocks from a seeded permuted pool
  3  chunked-prefill append + gather: 32 layers, 8 sequences x 2048 new tokens
     into a pool fragmented by freeing a random 40% of its blocks
  4  long-context decode: 1 layer (timed x32), batch 16 at 32768 tokens, Q
     scaled by 3 so the logits have std ~3
  5  swap under load (OLMoE-shaped): 16 layers, Hkv = Hq = 16, batch 128 at
     2048 tokens, 25% of the sequences evicted and restored
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

PAGE = 16


@dataclass(frozen=True)
class KVShape:
    num_layers: int
    num_kv_heads: int
    num_qo_heads: int
    head_dim: int = 128
    page_size: int = PAGE

    @property
    def token_row_bytes(self) -> int:
        """K or V bytes of one token (all KV heads), bf16."""
        return self.num_kv_heads * self.head_dim * 2

    @property
    def block_bytes(self) -> int:
        return self.page_size * self.token_row_bytes


MIXTRAL = KVShape(num_layers=32, num_kv_heads=8, num_qo_heads=32)
OLMOE = KVShape(num_layers=16, num_kv_heads=16, num_qo_heads=16)


def generator(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def randn_bf16(shape, seed: int, std: float = 1.0) -> torch.Tensor:
    """N(0, std^2) drawn in fp32 on the CPU, rounded to bf16."""
    x = torch.randn(*shape, generator=generator(seed), dtype=torch.float32)
    if std != 1.0:
        x = x * std
    return x.to(torch.bfloat16)


def randperm(n: int, seed: int) -> list[int]:
    return torch.randperm(n, generator=generator(seed)).tolist()


def uniform_ints(lo: int, hi: int, n: int, seed: int) -> list[int]:
    """n integers uniform in [lo, hi] inclusive."""
    return torch.randint(lo, hi + 1, (n,), generator=generator(seed)).tolist()


# ----------------------------------------------------------------- configs
@dataclass
class Config:
    name: str
    shape: KVShape
    seq_lens: list[int]                  # tokens resident before the step
    total_pages: int
    free_order: list[int]
    new_tokens: int = 1                  # tokens appended per sequence per step
    q_std: float = 1.0
    extra: dict = field(default_factory=dict)


def config1(seed: int = 0) -> Config:
    shape = KVShape(num_layers=2, num_kv_heads=8, num_qo_heads=32)
    return Config("cfg1-small", shape, [37, 128, 255, 513], 256, randperm(256, seed + 1))


def config2(seed: int = 0, batch: int = 64, extra_steps: int = 64) -> Config:
    lens = uniform_ints(512, 4096, batch, seed + 2)
    pages = sum((ln + extra_steps + PAGE - 1) // PAGE for ln in lens) + batch
    return Config("cfg2-mixtral-decode", MIXTRAL, lens, pages, randperm(pages, seed + 3),
                  extra={"extra_steps": extra_steps})


def config3(seed: int = 0, pool_blocks: int = 4096, frac_freed: float = 0.4) -> Config:
    """8 sequences x 2048 new tokens into a pool whose free list is a seeded
    random 40% of its blocks (in random order)."""
    freed = randperm(pool_blocks, seed + 4)[: int(round(frac_freed * pool_blocks))]
    return Config("cfg3-chunked-prefill", MIXTRAL, [0] * 8, pool_blocks, freed,
                  new_tokens=2048, extra={"fragmented_free": freed})


def config4(seed: int = 0) -> Config:
    shape = KVShape(num_layers=1, num_kv_heads=8, num_qo_heads=32)
    lens = [32768] * 16
    pages = sum((ln + PAGE) // PAGE + 1 for ln in lens)
    return Config("cfg4-long-context", shape, lens, pages, randperm(pages, seed + 5),
                  q_std=3.0, extra={"timed_repeats": 32})


def config5(seed: int = 0) -> Config:
    lens = [2048] * 128
    pages = 16384
    return Config("cfg5-olmoe-swap", OLMOE, lens, pages, randperm(pages, seed + 6),
                  extra={"swap_fraction": 0.25})


# ------------------------------------------------------------- byte counts
def decode_bytes(ctx_lens, num_qo_heads: int, num_kv_heads: int, head_dim: int = 128,
                 page_size: int = PAGE, elem: int = 2) -> int:
    """Algorithmic HBM bytes of one decode-attention launch: every K and V row
    of every KV head read once, q read, out written, page ids read.  Split-K
    scratch traffic is excluded."""
    ctx = np.asarray(ctx_lens, dtype=np.int64)
    pages = int(((ctx + page_size - 1) // page_size).sum())
    return (int(ctx.sum()) * 2 * num_kv_heads * head_dim * elem
            + len(ctx) * num_qo_heads * head_dim * elem * 2 + 4 * pages)


def append_bytes(num_tokens: int, num_kv_heads: int, head_dim: int = 128, elem: int = 2) -> int:
    """K and V rows read and written once, plus the int64 slot."""
    return num_tokens * (2 * num_kv_heads * head_dim * elem) * 2 + 8 * num_tokens


def gather_bytes(seq_lens, num_kv_heads: int, head_dim: int = 128, page_size: int = PAGE,
                 elem: int = 2) -> int:
    """K and V rows read and written once, plus the block-table entries."""
    lens = np.asarray(seq_lens, dtype=np.int64)
    blocks = int(((lens + page_size - 1) // page_size).sum())
    return int(lens.sum()) * (2 * num_kv_heads * head_dim * elem) * 2 + 4 * blocks
