"""The forward context the attention path reads at call time.

Same fields, defaults, dtypes and module-global get / set / reset functions as the reference's
(reference: nanovllm_voxcpm/engine/utils.py:25-38 Context, :71-99 get_context / set_context, :161-163
reset_context), so a runner that sets the context for the reference's Attention sets it for this one:

- ``is_prefill`` bool; ``cu_seqlens_q`` / ``cu_seqlens_k`` int32 [B + 1]; ``max_seqlen_q`` / ``max_seqlen_k`` host ints;
- ``slot_mapping`` int32 [N] (-1 = padded row); ``context_lens`` int32 [B]; ``block_tables`` int32 [B, max_blocks]
  (-1 padded);
- ``first_patch``: carried for the reference's runner, not read by attention.

The context is a module global read when ``Attention.forward`` runs: callers such as the reference's ``last_rows``
(reference: nanovllm_voxcpm/kernels/fused_layer.py:767-773) mutate ``cu_seqlens_q`` / ``max_seqlen_q`` in place
around one call.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class Context:
    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    first_patch: bool = True


_CONTEXT = Context()


def get_context() -> Context:
    return _CONTEXT


def set_context(
    is_prefill,
    cu_seqlens_q=None,
    cu_seqlens_k=None,
    max_seqlen_q=0,
    max_seqlen_k=0,
    slot_mapping=None,
    context_lens=None,
    block_tables=None,
):
    global _CONTEXT
    _CONTEXT = Context(
        is_prefill,
        cu_seqlens_q,
        cu_seqlens_k,
        max_seqlen_q,
        max_seqlen_k,
        slot_mapping,
        context_lens,
        block_tables,
    )


def reset_context():
    global _CONTEXT
    _CONTEXT = Context()
