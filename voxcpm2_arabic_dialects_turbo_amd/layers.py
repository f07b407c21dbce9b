"""The drop-in attention module of the VoxCPM2 engine's causal and non-causal layers.

``Attention`` keeps the reference module's constructor, public attributes (``num_heads``, ``head_dim``, ``scale``,
``num_kv_heads``, ``is_causal`` and the assignable ``k_cache`` / ``v_cache`` that a runner sets to per-layer views
``kv[i, 0]`` / ``kv[i, 1]`` of one [layers, 2, num_blocks, block_size, HK, head_dim] allocation) and its
``forward(q, k, v)`` dispatch, reading the forward context at call time
(reference: nanovllm_voxcpm/model/layers.py:308-362):

- causal, caches allocated: store this step's K/V at ``slot_mapping`` first (in a decode step, inside the decode
  call itself: the same result without the store's own launch);
- causal prefill: varlen attention over the step's own k / v, or over the caches when ``block_tables`` is set
  (prefix cache, mixed prefill + decode steps, prefill graphs), bottom-right causal;
- causal decode: paged split-KV decode over ``context_lens`` / ``block_tables``; returns [B, 1, H, D];
- non-causal: dense attention over [B, L, H, D] (LocEnc / LocDiT rows).

Every branch runs a HIP kernel of libvoxattn.so; nothing here synchronizes or allocates outside torch, so the
module can be captured into HIP graphs exactly where the reference captures its decode step.
"""

from __future__ import annotations

import itertools
import os

import torch
from torch import nn

from .context import get_context
from .ops import (decode_attention, flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache, planning,
                  prefill_attention_store, store_kvcache)

__all__ = ["Attention", "store_kvcache"]


def _store_rides_in_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, slot_mapping) -> bool:
    """Whether a decode step's KV store can ride in the decode call (vox_decode_attn_store): one row per sequence
    and one slot per row, rows 16-byte aligned with heads contiguous and row strides a multiple of 8 elements (the
    decode kernel reads the new rows with 16-byte loads). Any other layout takes store_kvcache, whose element path
    copies unaligned rows, followed by the decode kernel: the same result."""
    if slot_mapping is None or k.dim() != 3 or v.dim() != 3 or k.shape[0] != q.shape[0] or v.shape != k.shape:
        return False
    if slot_mapping.numel() != q.shape[0]:
        return False
    for t in (k, v):
        if t.stride(2) != 1 or t.stride(1) != t.shape[2] or t.stride(0) % 8 or t.data_ptr() % 16 \
                or t.stride(0) < t.shape[1] * t.shape[2]:
            return False
    return True


def _store_rides_in_prefill(k: torch.Tensor, v: torch.Tensor, slot_mapping) -> bool:
    """Whether a prefill step's KV store can ride in its attention call (prefill_attention_store): [N, HK, D] key and
    value rows with heads contiguous and one slot per row. (The library itself takes the store and the attention as
    two launches where its copy cannot move the rows.) Any other layout takes store_kvcache then the attention."""
    if slot_mapping is None or k.dim() != 3 or v.shape != k.shape or slot_mapping.numel() != k.shape[0]:
        return False
    return all(t.stride(2) == 1 and t.stride(1) == t.shape[2] for t in (k, v))


def _check_riding_store(context, block_size: int, decode: bool) -> None:
    """With VOX_CHECK_STORE=1 in the environment: verify on the host that this step's slots are those its block tables
    give the new tokens and that no new slot lies in another sequence's context, which the riding stores assume
    (checks.py); raise ValueError otherwise. Off by default (it copies the context to the host and synchronizes)."""
    if os.environ.get("VOX_CHECK_STORE") != "1" or context.block_tables is None:
        return
    from .checks import riding_store_violations

    v = riding_store_violations(context.slot_mapping, context.block_tables, block_size,
                                context_lens=context.context_lens if decode else None,
                                cu_seqlens_q=None if decode else context.cu_seqlens_q,
                                cu_seqlens_k=None if decode else context.cu_seqlens_k)
    if v:
        raise ValueError("riding KV store: the step's slots break its assumptions: " + "; ".join(v))


_PLAN_SERIAL = itertools.count(1)


def _plan_key(context) -> tuple:
    """The decode-plan key of a forward context: one serial per context object (a new set_context is a new step) and
    the tensors the layout is read from, so every layer of a step shares one plan and a context whose tensors are
    swapped (last_rows) records its own."""
    serial = context.__dict__.get("_vox_plan_serial")
    if serial is None:
        serial = next(_PLAN_SERIAL)
        context._vox_plan_serial = serial

    def ident(t):
        return None if t is None else (t.data_ptr(), tuple(t.shape), tuple(t.stride()))

    return (serial, ident(context.context_lens), ident(context.block_tables), ident(context.slot_mapping),
            ident(context.cu_seqlens_q), ident(context.cu_seqlens_k))


class Attention(nn.Module):

    def __init__(
        self,
        num_heads,
        head_dim,
        scale,
        num_kv_heads,
        is_causal: bool = True,
    ):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.k_cache = self.v_cache = torch.tensor([])
        self.is_causal = is_causal

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
        if self.is_causal:
            context = get_context()
            k_cache, v_cache = self.k_cache, self.v_cache
            cached = bool(k_cache.numel() and v_cache.numel())
            if cached and not context.is_prefill and _store_rides_in_decode(q, k, v, context.slot_mapping):
                # decode step: the store rides in the decode call (one row per sequence, each writing the slot of
                # its own newest token)
                _check_riding_store(context, k_cache.shape[1], decode=True)
                return decode_attention(q, k_cache, v_cache, context.context_lens, context.block_tables, self.scale,
                                        key=k, value=v, slot_mapping=context.slot_mapping,
                                        plan=_plan_key(context)).unsqueeze(1)
            if cached and context.is_prefill and context.cu_seqlens_q is not None \
                    and _store_rides_in_prefill(k, v, context.slot_mapping):
                # prefill: the store rides in the attention call. Over the step's own rows (no block table) the
                # launch reads the packed rows; through the block tables (prefix cache, mixed steps) the launch reads
                # each sequence's new keys from the rows and writes the caches after its reads
                bt = context.block_tables
                _check_riding_store(context, k_cache.shape[1], decode=False)
                return prefill_attention_store(q, k, v, k_cache, v_cache, context.slot_mapping,
                                               cu_seqlens_q=context.cu_seqlens_q, cu_seqlens_k=context.cu_seqlens_k,
                                               max_seqlen_q=context.max_seqlen_q, softmax_scale=self.scale,
                                               causal=True, block_table=bt,
                                               plan=_plan_key(context) if bt is not None else None)
            if cached:
                store_kvcache(k, v, k_cache, v_cache, context.slot_mapping)
            if context.is_prefill:
                if context.block_tables is not None:  # prefix cache: keys through the block tables
                    k, v = k_cache, v_cache
                # (a mixed step's one-query rows run on the decode kernel: their layout is planned per context)
                with planning(_plan_key(context) if context.block_tables is not None else None):
                    o = flash_attn_varlen_func(
                        q,
                        k,
                        v,
                        max_seqlen_q=context.max_seqlen_q,
                        cu_seqlens_q=context.cu_seqlens_q,
                        max_seqlen_k=context.max_seqlen_k,
                        cu_seqlens_k=context.cu_seqlens_k,
                        softmax_scale=self.scale,
                        causal=True,
                        block_table=context.block_tables,
                    )
            else:  # decode
                o = flash_attn_with_kvcache(
                    q.unsqueeze(1),
                    k_cache,
                    v_cache,
                    cache_seqlens=context.context_lens,
                    block_table=context.block_tables,
                    softmax_scale=self.scale,
                    causal=True,
                )
        else:  # non-causal, no KV cache
            o = flash_attn_func(q, k, v, softmax_scale=self.scale, causal=False)
        return o
