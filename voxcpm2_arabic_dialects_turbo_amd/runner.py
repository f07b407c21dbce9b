"""Host side of the attention path: KV-cache allocation, the per-step attention context, decode graph buffers.

These produce exactly the tensors the reference's runner hands to Attention.forward, with the same values, dtypes
and shapes (reference: nanovllm_voxcpm/engine/model_runner.py):

- ``allocate_kv_cache``: one [layers, 2, num_blocks, block_size, HK, head_dim] allocation; causal layer i gets the
  views ``kv[i, 0]`` / ``kv[i, 1]`` (reference :679-751, layout :728-737).
- ``prepare_decode_context``: positions int64 = len - 1, slot_mapping int32 = table[-1] * block_size +
  last_block_num_tokens - 1, context_lens int32 = len, block_tables int32 padded with -1 (reference :913-938,
  :841-844).
- ``stage_prefill_context`` / ``prepare_prefill_context``: positions int64 of the uncached tokens, cu_seqlens_q/k
  int32, host max lengths, token-granular slot_mapping int32, block_tables int32 when there is a cached prefix
  (cu_seqlens_k[-1] > cu_seqlens_q[-1]) or when prefill graphs read keys through tables (reference :851-911),
  computed with numpy in one pass per array and uploaded in one H2D copy from one page-locked buffer
  (``HostPack``, reference :237-297).
- ``DecodeGraphBuffers``: the static decode buffers a captured graph reads; loading a step fills slot_mapping
  with -1 and context_lens with 0 past the batch and overwrites the first columns of block_tables, leaving stale
  columns (reference :1150-1152, :1558-1566). The decode kernel never reads a column past a row's context.
"""

from __future__ import annotations

import math
from typing import Callable, Iterable

import numpy as np
import torch

from .context import get_context, set_context
from .layers import Attention

_TORCH_DTYPES = {np.dtype(np.int64): torch.int64, np.dtype(np.int32): torch.int32,
                 np.dtype(np.float32): torch.float32, np.dtype(np.uint8): torch.uint8}


class RunnerTask:
    """What the runner knows of one sequence in a step (reference: nanovllm_voxcpm/engine/model_runner.py:140-165)."""

    def __init__(self, block_table: list[int], seq_length: int, num_cached_tokens: int, block_size: int,
                 seq_id: str | None = None):
        self.block_table = block_table
        self.seq_length = seq_length
        self.num_cached_tokens = num_cached_tokens
        self.block_size = block_size
        self.seq_id = seq_id

    @property
    def num_blocks(self) -> int:
        return (self.seq_length + self.block_size - 1) // self.block_size

    @property
    def last_block_num_tokens(self) -> int:
        return self.seq_length - (self.num_blocks - 1) * self.block_size


class HostPack:
    """A step's host arrays staged in one buffer and copied to the device in one transfer. ``add`` returns the index
    of the tensor ``upload`` hands back: a view of the one device buffer with the array's dtype, shape and values.
    Parts start at multiples of 256 bytes."""

    ALIGN = 256

    def __init__(self, device="cuda"):
        self.device = torch.device(device)
        self.parts: list[np.ndarray] = []

    def add(self, array) -> int:
        self.parts.append(np.asarray(array))
        return len(self.parts) - 1

    def upload(self) -> list[torch.Tensor]:
        offsets, total = [], 0
        for a in self.parts:
            offsets.append(total)
            total += -(-a.nbytes // self.ALIGN) * self.ALIGN
        total = max(total, self.ALIGN)
        on_gpu = self.device.type == "cuda"
        host = torch.empty(total, dtype=torch.uint8, pin_memory=on_gpu)
        buf = host.numpy()
        for a, off in zip(self.parts, offsets):
            buf[off:off + a.nbytes] = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
        dev = host.to(self.device, non_blocking=True) if on_gpu else host
        out = []
        for a, off in zip(self.parts, offsets):
            t = dev[off:off + a.nbytes].view(_TORCH_DTYPES[a.dtype])
            out.append(t.view(a.shape) if a.ndim != 1 else t)
        return out


def block_tables_array(seqs: list[RunnerTask]) -> np.ndarray:
    """int32 [n, max_blocks], rows padded with -1 (reference: nanovllm_voxcpm/engine/model_runner.py:841-844)."""
    n = len(seqs)
    lens = [len(s.block_table) for s in seqs]
    m = max(lens, default=0)
    tables = np.full((n, m), -1, dtype=np.int32)
    for i, s in enumerate(seqs):
        tables[i, :lens[i]] = s.block_table
    return tables


def stage_prefill_context(seqs: list[RunnerTask], block_size: int, pack: HostPack, graphs: bool = False
                          ) -> Callable[[list[torch.Tensor]], torch.Tensor]:
    """Stages the prefill context of ``seqs`` in ``pack``; returns ``finish(uploaded)`` that sets the context from
    the uploaded views and returns the positions (reference: nanovllm_voxcpm/engine/model_runner.py:851-911)."""
    n = len(seqs)
    seqlen_k = np.fromiter((s.seq_length for s in seqs), dtype=np.int64, count=n)
    cached = np.fromiter((s.num_cached_tokens for s in seqs), dtype=np.int64, count=n)
    seqlen_q = seqlen_k - cached
    cu_q = np.zeros(n + 1, dtype=np.int64)
    cu_k = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(seqlen_q, out=cu_q[1:])
    np.cumsum(seqlen_k, out=cu_k[1:])
    max_q = int(seqlen_q.max(initial=0))
    max_k = int(seqlen_k.max(initial=0))
    total_q = int(cu_q[-1])
    seq_of_token = np.repeat(np.arange(n), seqlen_q)
    positions = np.arange(total_q, dtype=np.int64) - np.repeat(cu_q[:-1] - cached, seqlen_q)
    tables = block_tables_array(seqs).astype(np.int64)
    has_table = np.array([len(s.block_table) > 0 for s in seqs], dtype=bool)
    with_table = has_table[seq_of_token] if total_q else np.zeros(0, dtype=bool)
    tok_seq, tok_pos = seq_of_token[with_table], positions[with_table]
    slots = tables[tok_seq, tok_pos // block_size] * block_size + tok_pos % block_size if tok_seq.size \
        else np.zeros(0, np.int64)
    i_pos = pack.add(positions)
    i_cu_q = pack.add(cu_q.astype(np.int32))
    i_cu_k = pack.add(cu_k.astype(np.int32))
    i_slot = pack.add(slots.astype(np.int32))
    i_bt = pack.add(tables.astype(np.int32)) if (cu_k[-1] > cu_q[-1] or graphs) else None

    def finish(views: list[torch.Tensor]) -> torch.Tensor:
        set_context(True, views[i_cu_q], views[i_cu_k], max_q, max_k, views[i_slot], None,
                    views[i_bt] if i_bt is not None else None)
        return views[i_pos]

    return finish


def prepare_prefill_context(seqs: list[RunnerTask], block_size: int, device="cuda", graphs: bool = False
                            ) -> torch.Tensor:
    pack = HostPack(device)
    finish = stage_prefill_context(seqs, block_size, pack, graphs=graphs)
    return finish(pack.upload())


def prepare_decode_context(seqs: list[RunnerTask], block_size: int, device="cuda") -> torch.Tensor:
    """Sets the decode context of ``seqs`` and returns the positions (reference:
    nanovllm_voxcpm/engine/model_runner.py:913-938)."""
    n = len(seqs)
    lens = np.fromiter((s.seq_length for s in seqs), dtype=np.int64, count=n)
    last_block = np.fromiter((s.block_table[-1] for s in seqs), dtype=np.int64, count=n)
    nblk = (lens + block_size - 1) // block_size
    last_tokens = lens - (nblk - 1) * block_size
    pack = HostPack(device)
    i_pos = pack.add(lens - 1)
    i_slot = pack.add((last_block * block_size + last_tokens - 1).astype(np.int32))
    i_len = pack.add(lens.astype(np.int32))
    i_bt = pack.add(block_tables_array(seqs))
    views = pack.upload()
    set_context(False, slot_mapping=views[i_slot], context_lens=views[i_len], block_tables=views[i_bt])
    return views[i_pos]


def causal_attention_modules(model: torch.nn.Module) -> list[Attention]:
    return [m for m in model.modules() if isinstance(m, Attention) and m.is_causal]


def kv_cache_block_bytes(modules: Iterable[Attention], block_size: int, dtype=torch.bfloat16) -> int:
    """Bytes one cache block takes across every causal layer, K and V (reference: model_runner.py:680-686)."""
    itemsize = torch.empty(0, dtype=dtype).element_size()
    return sum(2 * block_size * m.num_kv_heads * m.head_dim * itemsize for m in modules)


def allocate_kv_cache(model_or_modules, num_blocks: int, block_size: int, dtype=torch.bfloat16, device="cuda"
                      ) -> torch.Tensor | None:
    """Allocates the KV cache and assigns every causal Attention its per-layer views. One
    [layers, 2, num_blocks, block_size, HK, head_dim] tensor when all layers share a head shape (a block's KV across
    all layers is then reachable from one base pointer), else one pair of tensors per layer
    (reference: nanovllm_voxcpm/engine/model_runner.py:726-751)."""
    if num_blocks <= 0:
        raise ValueError("num_blocks must be positive")
    if block_size % 256:
        raise ValueError("kvcache_block_size must be a multiple of 256")  # reference: engine/config.py:27
    modules = causal_attention_modules(model_or_modules) if isinstance(model_or_modules, torch.nn.Module) \
        else list(model_or_modules)
    shapes = {(m.num_kv_heads, m.head_dim) for m in modules}
    if len(shapes) == 1:
        heads, dim = shapes.pop()
        kv = torch.empty(len(modules), 2, num_blocks, block_size, heads, dim, dtype=dtype, device=device)
        for i, m in enumerate(modules):
            m.k_cache, m.v_cache = kv[i, 0], kv[i, 1]
        return kv
    for m in modules:
        m.k_cache = torch.empty(num_blocks, block_size, m.num_kv_heads, m.head_dim, dtype=dtype, device=device)
        m.v_cache = torch.empty(num_blocks, block_size, m.num_kv_heads, m.head_dim, dtype=dtype, device=device)
    return None


class DecodeGraphBuffers:
    """Static decode-context buffers that a captured decode graph reads (reference:
    nanovllm_voxcpm/engine/model_runner.py:1150-1152 allocation, :1558-1566 per-step load)."""

    def __init__(self, max_bs: int, max_num_blocks: int, device="cuda"):
        self.max_bs = max_bs
        self.slot_mapping = torch.zeros(max_bs, dtype=torch.int32, device=device)
        self.context_lens = torch.zeros(max_bs, dtype=torch.int32, device=device)
        self.block_tables = torch.zeros(max_bs, max_num_blocks, dtype=torch.int32, device=device)

    def bind(self, bs: int) -> None:
        """Sets the decode context to the first ``bs`` rows of the static buffers (done before capture)."""
        set_context(False, slot_mapping=self.slot_mapping[:bs], context_lens=self.context_lens[:bs],
                    block_tables=self.block_tables[:bs])

    def load(self, bs: int | None = None) -> None:
        """Copies the current (eager-built) decode context into the static buffers, as run_model does."""
        ctx = get_context()
        n = ctx.context_lens.numel() if bs is None else bs
        self.slot_mapping.fill_(-1)
        self.slot_mapping[:n] = ctx.slot_mapping
        self.context_lens.zero_()
        self.context_lens[:n] = ctx.context_lens
        self.block_tables[:n, :ctx.block_tables.size(1)] = ctx.block_tables


def graph_batch_sizes(max_bs: int) -> list[int]:
    """The captured decode batch sizes (reference: nanovllm_voxcpm/engine/model_runner.py:1161-1162)."""
    cands = [1, 2, 4, 8] + list(range(16, max_bs + 1, 16)) + [max_bs]
    return sorted({bs for bs in cands if 1 <= bs <= max_bs})


def num_blocks_for(max_model_len: int, block_size: int) -> int:
    return math.ceil(max_model_len / block_size)
