"""Shared input generators and tolerance checks for the parity tests (not a test module)."""

from __future__ import annotations

import torch

H, HK, D = 16, 2, 128
BLOCK = 256

# north-star tolerances for bf16 attention outputs with fp32 accumulation
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def randn(gen: torch.Generator, *shape, dtype=torch.bfloat16) -> torch.Tensor:
    """N(0, 1) values from a seeded CPU generator, rounded to ``dtype`` (CPU tensor)."""
    return torch.randn(*shape, generator=gen, dtype=torch.float32).to(dtype)


def attn_close(out: torch.Tensor, ref: torch.Tensor, what: str = "", max_abs: float = MAX_ABS,
               mean_abs: float = MEAN_ABS) -> tuple[float, float]:
    """Asserts max|out - ref| <= max_abs and mean|out - ref| <= mean_abs (out bf16 on any device, ref fp32/fp64)."""
    diff = (out.detach().float().cpu() - ref.float().cpu()).abs()
    assert torch.isfinite(out.float().cpu()).all(), f"{what}: non-finite output"
    mx, mn = diff.max().item() if diff.numel() else 0.0, diff.mean().item() if diff.numel() else 0.0
    assert mx <= max_abs and mn <= mean_abs, f"{what}: max-abs {mx:.3g} (<= {max_abs}), mean-abs {mn:.3g} (<= {mean_abs})"
    return mx, mn


def paged_pool(gen: torch.Generator, lens: list[int], pool: int, block_size: int = BLOCK, hk: int = HK,
               d: int = D, extra_cols: int = 0):
    """Random caches [pool, block_size, hk, d] (bf16, CPU) and non-overlapping block tables drawn from
    randperm(pool), padded with -1 (plus ``extra_cols`` trailing -1 columns)."""
    k_cache = randn(gen, pool, block_size, hk, d)
    v_cache = randn(gen, pool, block_size, hk, d)
    perm = torch.randperm(pool, generator=gen).tolist()
    need = [(n + block_size - 1) // block_size for n in lens]
    assert sum(need) <= pool, "pool too small"
    width = max(need + [1]) + extra_cols
    tables = torch.full((len(lens), width), -1, dtype=torch.int32)
    at = 0
    for i, nb in enumerate(need):
        tables[i, :nb] = torch.tensor(perm[at:at + nb], dtype=torch.int32)
        at += nb
    return k_cache, v_cache, tables


def uniform_lens(gen: torch.Generator, n: int, lo: int, hi: int) -> list[int]:
    return torch.randint(lo, hi + 1, (n,), generator=gen).tolist()
