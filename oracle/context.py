"""Per-token definitions of the attention context tensors (test infrastructure only; see oracle/__init__.py).

``prefill_context`` restates the per-token loop the reference's test suite keeps as the definition of the prefill
context (reference: tests/test_burst_host_path.py:87-107, ``_old_prefill_context``); ``decode_context`` restates
the decode builder's per-sequence formulas (reference: nanovllm_voxcpm/engine/model_runner.py:913-938 with the -1
padded block tables of :841-844). A task needs ``block_table`` (list of ints), ``seq_length`` and
``num_cached_tokens``.
"""

from __future__ import annotations


def prefill_context(block_size: int, seqs, graphs: bool = False):
    """Returns (positions, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, slot_mapping, block_tables or
    None) as Python lists / ints, one token at a time."""
    positions, cu_q, cu_k, max_q, max_k, slots = [], [0], [0], 0, 0, []
    for seq in seqs:
        seq_len = seq.seq_length
        positions.extend(range(seq.num_cached_tokens, seq_len))
        nq = seq_len - seq.num_cached_tokens
        cu_q.append(cu_q[-1] + nq)
        cu_k.append(cu_k[-1] + seq_len)
        max_q, max_k = max(nq, max_q), max(seq_len, max_k)
        if not seq.block_table:  # warm-up tasks: no cache, no slots
            continue
        for pos in range(seq.num_cached_tokens, seq_len):
            slots.append(seq.block_table[pos // block_size] * block_size + pos % block_size)
    tables = None
    if cu_k[-1] > cu_q[-1] or graphs:
        m = max(len(s.block_table) for s in seqs)
        tables = [s.block_table + [-1] * (m - len(s.block_table)) for s in seqs]
    return positions, cu_q, cu_k, max_q, max_k, slots, tables


def decode_context(block_size: int, seqs):
    """Returns (positions, slot_mapping, context_lens, block_tables) as Python lists: the new token of each sequence
    sits at position seq_length - 1, in the last block at offset last_block_num_tokens - 1."""
    positions, slots, lens = [], [], []
    for seq in seqs:
        num_blocks = (seq.seq_length + block_size - 1) // block_size
        last_block_tokens = seq.seq_length - (num_blocks - 1) * block_size
        positions.append(seq.seq_length - 1)
        lens.append(seq.seq_length)
        slots.append(seq.block_table[-1] * block_size + last_block_tokens - 1)
    m = max(len(s.block_table) for s in seqs)
    tables = [s.block_table + [-1] * (m - len(s.block_table)) for s in seqs]
    return positions, slots, lens, tables
