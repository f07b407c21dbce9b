"""CPU restatement of the KV block-prefix copy (test infrastructure only; see oracle/__init__.py)."""

from __future__ import annotations

import torch


def copy_kv_block_prefix(kv: torch.Tensor, entries) -> None:
    """In place on kv [layers, 2, blocks, block_size, kv_heads, head_dim]: for each (src, dst, n) with n > 0,
    kv[:, :, dst, :min(n, block_size)] = kv[:, :, src, :min(n, block_size)], entries applied in order.
    Reference: nanovllm_voxcpm/kernels/kv_copy.py:17-41 (one launch; entries that do not overlap give the same
    result in any order)."""
    block_size = kv.shape[3]
    for src, dst, n in entries:
        n = min(int(n), block_size)
        if n <= 0:
            continue
        kv[:, :, dst, :n] = kv[:, :, src, :n].clone()
