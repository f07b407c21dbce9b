"""Short-sequence attention with the reference's Triton-kernel interfaces, on the HIP varlen kernel.

- ``short_causal_attention``: varlen causal attention of a prefill step's short sequences over their own tokens
  (reference: nanovllm_voxcpm/kernels/short_attn.py:156-179): q [T, H, D], k / v [T, HK, D] (token rows may be strided
  views of the qkv output), cu_seqlens [B + 1], 0 < max_seqlen <= SHORT_CAUSAL_MAX_LEN. Returns o [T, H * D].
- ``short_attention``: non-causal attention of LocEnc / LocDiT rows (reference: kernels/short_attn.py:70-90):
  q [B, L, H, D], k / v [B, L, HK, D]. Returns o [B * L, H * D].

Both keep the reference's argument checks. With ``quant`` they return (int8 o, fp32 per-token scale): o * inv_smooth
quantized per token over all heads in the kernel's epilogue (reference: kernels/short_attn.py:55-64, 137-146).
"""

from __future__ import annotations

import torch

from ..ops import _token_rows, varlen_attention

# the longest sequence the reference's short causal kernel takes (one 32-token tile per sequence)
SHORT_CAUSAL_MAX_LEN = 32


def short_causal_attention(q, k, v, cu_seqlens, max_seqlen: int, sm_scale: float, quant: bool = False,
                           inv_smooth=None):
    T, H, D = q.shape
    HK = k.shape[1]
    assert q.stride(2) == 1 and q.stride(1) == D and k.stride(1) == D and k.stride() == v.stride()
    assert 0 < max_seqlen <= SHORT_CAUSAL_MAX_LEN
    assert H % HK == 0
    if quant:
        return varlen_attention(q, k, v, cu_seqlens_q=cu_seqlens, cu_seqlens_k=cu_seqlens, max_seqlen_q=max_seqlen,
                                softmax_scale=sm_scale, causal=True, quant=True, inv_smooth=inv_smooth)
    o = torch.empty(T, H * D, device=q.device, dtype=q.dtype)
    varlen_attention(q, k, v, cu_seqlens_q=cu_seqlens, cu_seqlens_k=cu_seqlens, max_seqlen_q=max_seqlen,
                     softmax_scale=sm_scale, causal=True, out=o.view(T, H, D))
    return o


def short_attention(q, k, v, sm_scale: float, quant: bool = False, inv_smooth=None, num_warps: int = 4):
    B, L, H, D = q.shape
    HK = k.shape[2]
    assert q.stride(3) == 1 and q.stride(2) == D and k.stride(2) == D and k.stride() == v.stride()
    args = dict(cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=L, softmax_scale=sm_scale, causal=False,
                batch=B, uniform_seqlen_q=L, uniform_seqlen_k=L)
    if quant:
        return varlen_attention(_token_rows(q), _token_rows(k), _token_rows(v), quant=True, inv_smooth=inv_smooth,
                                **args)
    o = torch.empty(B * L, H * D, device=q.device, dtype=q.dtype)
    varlen_attention(_token_rows(q), _token_rows(k), _token_rows(v), out=o.view(B * L, H, D), **args)
    return o
