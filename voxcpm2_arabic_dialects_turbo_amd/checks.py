"""Host-side check of what the riding KV stores assume about a step's slots (a debugging aid, not the hot path).

A decode step's store riding in the decode call (vox_decode_attn_store), and a paged prefill or mixed step's store
riding in its attention launch (vox_prefill_attn_store_paged; vox_prefill_attn_int8_store with block tables), read
each sequence's new keys from the step's key / value rows instead of the cache, and write the cache after their
reads. The result equals store_kvcache followed by the
attention when

1. each sequence's new tokens have the slots its block table gives their positions,
   slot = block_tables[b, pos // block_size] * block_size + pos % block_size (a decode row's new token at position
   context_lens[b] - 1; a varlen sequence's nq new tokens at positions nk - nq .. nk - 1), and
2. no sequence's new slot lies inside another sequence's context (the slots its table gives positions 0 .. nk - 1),

which the reference engine guarantees: its runner computes the slots from the tables exactly so
(nanovllm_voxcpm/engine/model_runner.py:880-883 for prefill, :919 for decode) and its block manager gives every
sequence's last block to that sequence alone. `riding_store_violations` checks both on the host for one step's
context, so an integration that builds its own contexts can verify them; ``Attention.forward`` runs it before every
riding store when the environment sets ``VOX_CHECK_STORE=1`` (it copies the context to the host and synchronizes).
"""

from __future__ import annotations

import numpy as np
import torch

__all__ = ["riding_store_violations"]


def _host(t: torch.Tensor | None) -> np.ndarray | None:
    return None if t is None else t.detach().to("cpu", torch.int64).numpy()


def riding_store_violations(slot_mapping: torch.Tensor, block_tables: torch.Tensor, block_size: int, *,
                            context_lens: torch.Tensor | None = None, cu_seqlens_q: torch.Tensor | None = None,
                            cu_seqlens_k: torch.Tensor | None = None, limit: int = 10) -> list[str]:
    """The violations of the two conditions above in one step (at most `limit` messages; empty when both hold).
    Decode steps give context_lens (one new token per sequence, slot_mapping[b]); prefill and mixed steps give
    cu_seqlens_q / cu_seqlens_k (slot_mapping indexed by token row)."""
    slots, tables = _host(slot_mapping).reshape(-1), _host(block_tables)
    if tables is None or tables.ndim != 2:
        return ["no block tables: the riding stores need them"]
    if context_lens is not None:
        nk = _host(context_lens).reshape(-1)
        nq = np.ones_like(nk)
        row0 = np.arange(nk.size)
    elif cu_seqlens_q is not None and cu_seqlens_k is not None:
        cq, ck = _host(cu_seqlens_q).reshape(-1), _host(cu_seqlens_k).reshape(-1)
        nq, nk, row0 = np.diff(cq), np.diff(ck), cq[:-1]
    else:
        return ["give context_lens (decode) or cu_seqlens_q and cu_seqlens_k (prefill)"]
    out: list[str] = []
    batch, width = min(nk.size, tables.shape[0]), tables.shape[1]

    def slot_of(b: int, pos: np.ndarray) -> np.ndarray:
        col = pos // block_size
        ok = col < width
        blk = np.where(ok, tables[b, np.minimum(col, width - 1)], -1)
        return np.where(ok & (blk >= 0), blk * block_size + pos % block_size, -1)

    new_slots: dict[int, np.ndarray] = {}
    for b in range(batch):
        if nq[b] <= 0 or nk[b] <= 0:
            continue
        pos = np.arange(nk[b] - nq[b], nk[b])
        rows = row0[b] + np.arange(nq[b]) if context_lens is None else np.array([b])
        if rows[-1] >= slots.size:
            out.append(f"sequence {b}: rows {rows[0]}..{rows[-1]} past slot_mapping ({slots.size} slots)")
            continue
        want, got = slot_of(b, pos), slots[rows]
        bad = np.nonzero(got != want)[0]
        if bad.size:
            i = int(bad[0])
            out.append(f"sequence {b}: new token at position {int(pos[i])} has slot {int(got[i])}, its block table "
                       f"gives {int(want[i])} ({bad.size} such tokens)")
        new_slots[b] = got[got >= 0]
        if len(out) >= limit:
            return out
    owner = {}
    for b, s in new_slots.items():
        for v in s.tolist():
            owner[v] = b
    for b in range(batch):
        if nk[b] <= 0 or not owner:
            continue
        ctx = slot_of(b, np.arange(nk[b]))
        for v in ctx[ctx >= 0].tolist():
            o = owner.get(v)
            if o is not None and o != b:
                out.append(f"sequence {o}'s new slot {v} lies inside sequence {b}'s context")
                if len(out) >= limit:
                    return out
                break
    return out
