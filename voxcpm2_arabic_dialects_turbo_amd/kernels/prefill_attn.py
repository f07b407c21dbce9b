"""Paged causal prefill attention with the reference's Triton-kernel interface, on the HIP varlen kernel.

``paged_prefill_attention`` keeps the signature and output layout of the reference's function
(reference: nanovllm_voxcpm/kernels/prefill_attn.py:98-124): q [T, H, D] (token rows may be strided, e.g. a view of
the qkv GEMM output), the paged caches [pages, page, HK, D], block_table [B, *], cu_seqlens_q / cu_seqlens_k
[B + 1]; query t of a sequence with nq new tokens and nk keys sits at position nk - nq + t. Returns o [T, H * D] in
q's dtype, or with ``quant`` (int8 o [T, H * D], fp32 scale [T]): o * inv_smooth quantized per token over all heads
(reference: kernels/prefill_attn.py:84-92), computed in the kernel's epilogue from the fp32 o. The tile-shape knobs
(block_q, block_k, num_warps) of the Triton kernel are accepted and ignored: the HIP kernel's tiling is fixed for
gfx950.
"""

from __future__ import annotations

import torch

from ..ops import varlen_attention


def paged_prefill_attention(q, k_cache, v_cache, block_table, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int,
                            sm_scale: float, quant: bool = False, inv_smooth=None, block_q: int = 8,
                            block_k: int = 32, num_warps: int = 4):
    T, H, D = q.shape
    pages, page, HK, _ = k_cache.shape
    assert q.stride(2) == 1 and q.stride(1) == D and k_cache.is_contiguous() and v_cache.is_contiguous()
    assert H % HK == 0
    if quant:
        return varlen_attention(q, None, None, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k,
                                max_seqlen_q=max_seqlen_q, softmax_scale=sm_scale, causal=True,
                                block_table=block_table, k_cache=k_cache, v_cache=v_cache, quant=True,
                                inv_smooth=inv_smooth)
    o = torch.empty(T, H * D, device=q.device, dtype=q.dtype)
    varlen_attention(q, None, None, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k,
                     max_seqlen_q=max_seqlen_q, softmax_scale=sm_scale, causal=True, block_table=block_table,
                     k_cache=k_cache, v_cache=v_cache, out=o.view(T, H, D))
    return o
