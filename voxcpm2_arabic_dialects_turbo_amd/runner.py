"""Host side of the attention path: KV-cache allocation, the per-step attention context, decode graph buffers.

The producers hand ``Attention.forward`` exactly the tensors the reference's runner does, with the same values,
dtypes and shapes (reference: nanovllm_voxcpm/engine/model_runner.py; the per-token definitions the reference's
tests keep are restated in ``oracle.context`` and ``tests/test_host.py`` compares both):

- prefill (reference :851-911): positions int64 of the uncached tokens, cu_seqlens_q / cu_seqlens_k int32, host
  max lengths, token-granular slot_mapping int32, block_tables int32 (-1 padded) when a cached prefix exists or when
  prefill graphs read keys through tables;
- decode (reference :913-938, tables :841-844): positions int64 = len - 1, slot_mapping int32 = the new token's slot
  in the table's last block, context_lens int32 = len, block_tables int32 (-1 padded).

How they are built here. Every array is computed by whole-array numpy operations sized by sequences or by
(sequence, block) pieces, never by a Python loop over tokens: the token-level arrays (positions, slots) are
"segment ramps", concatenations of consecutive runs of integers produced by one cumulative sum over a step array
(``_runs``). Slots are consecutive inside one cache block, so a sequence's new tokens are a few runs, one per block
they touch. The arrays are written straight into a page-locked staging buffer laid out once per step
(``StepStaging``) and reach the device in one host-to-device copy.

- ``allocate_kv_cache``: one [layers, 2, num_blocks, block_size, HK, head_dim] allocation; causal layer i gets the
  views ``kv[i, 0]`` / ``kv[i, 1]`` (reference :679-751, layout :728-737).
- ``DecodeGraphBuffers``: the static decode buffers a captured graph reads; loading a step fills slot_mapping
  with -1 and context_lens with 0 past the batch and overwrites the first columns of block_tables, leaving stale
  columns (reference :1150-1152, :1558-1566). The decode kernel never uses a column past a row's context.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Iterable, Sequence

import numpy as np
import torch

from .context import get_context, set_context
from .layers import Attention


@dataclass
class RunnerTask:
    """One sequence of a step, as the scheduler hands it to the runner: its cache blocks, its length counting the
    tokens of this step, and how many of its leading tokens are already in the cache (the field contract of the
    reference's RunnerTask, nanovllm_voxcpm/engine/model_runner.py:140-165; any object with ``block_table``,
    ``seq_length`` and ``num_cached_tokens`` attributes is accepted by the producers below)."""

    block_table: list[int]
    seq_length: int
    num_cached_tokens: int
    block_size: int = 256
    seq_id: str | None = None


# ----------------------------------------------------------------------------------------------------------------------
# Page-locked staging


_ALIGN = 256  # every array starts at a multiple of 256 bytes, as separate device allocations would


@dataclass
class _Slot:
    host: torch.Tensor | None = None   # page-locked uint8 buffer
    done: object = None                # CUDA event recorded after the copy out of ``host``


@dataclass
class StepStaging:
    """Staging for one step's context arrays: ``layout`` reserves typed arrays at 256-byte offsets of one host
    buffer and returns numpy views to fill in place; ``upload`` copies the used bytes to the device in one
    transfer and returns torch views of the device copy with the same dtypes and shapes.

    On a GPU the host side is page-locked and persistent: two buffers alternate between steps, so the host can fill
    step n's arrays while step n - 1's copy may still be reading the other one; a buffer is refilled only after the
    event recorded behind its previous copy (normally long complete). A buffer grows (to twice the need) when a step
    needs more. Under graph capture, or on the CPU, a fresh buffer is used each time."""

    device: torch.device | str = "cuda"
    _slots: list[_Slot] = field(default_factory=lambda: [_Slot(), _Slot()])
    _turn: int = 0
    _host: torch.Tensor | None = None
    _slot: _Slot | None = None
    _parts: list[tuple[int, np.dtype, tuple]] = field(default_factory=list)
    _used: int = 0

    def layout(self, specs: Sequence[tuple[np.dtype, tuple]]) -> list[np.ndarray]:
        """Reserves one array per (dtype, shape) and returns writable numpy views of them (contents undefined)."""
        dev = torch.device(self.device)
        offsets, end = [], 0
        for dtype, shape in specs:
            dtype = np.dtype(dtype)
            offsets.append(end)
            end += -(-(dtype.itemsize * math.prod(shape)) // _ALIGN) * _ALIGN
        need = max(end, _ALIGN)
        persistent = dev.type == "cuda" and not torch.cuda.is_current_stream_capturing()
        if persistent:
            slot = self._slots[self._turn]
            self._turn ^= 1
            if slot.done is not None:
                slot.done.synchronize()
                slot.done = None
            if slot.host is None or slot.host.numel() < need:
                slot.host = torch.empty(2 * need, dtype=torch.uint8, pin_memory=True)
            self._host, self._slot = slot.host, slot
        else:
            self._host = torch.empty(need, dtype=torch.uint8, pin_memory=dev.type == "cuda")
            self._slot = None
        raw = self._host.numpy()
        self._parts, self._used = [], need
        views = []
        for off, (dtype, shape) in zip(offsets, specs):
            dtype = np.dtype(dtype)
            n = math.prod(shape)
            views.append(raw[off:off + n * dtype.itemsize].view(dtype).reshape(shape))
            self._parts.append((off, dtype, tuple(shape)))
        return views

    def upload(self) -> list[torch.Tensor]:
        """One copy of the laid-out bytes to the device (non-blocking from page-locked memory); the views."""
        dev = torch.device(self.device)
        src = self._host[:self._used]
        if dev.type == "cuda":
            dst = src.to(dev, non_blocking=True)
            if self._slot is not None:
                ev = torch.cuda.Event()
                ev.record()
                self._slot.done = ev
        else:
            dst = src.clone()
        out = []
        for off, dtype, shape in self._parts:
            n = math.prod(shape)
            t = dst[off:off + n * dtype.itemsize].view(_TORCH_DTYPE[dtype])
            out.append(t.view(shape))
        return out


_TORCH_DTYPE = {np.dtype(np.int64): torch.int64, np.dtype(np.int32): torch.int32}


# ----------------------------------------------------------------------------------------------------------------------
# Context producers


def _runs(first: np.ndarray, count: np.ndarray, out: np.ndarray | None = None) -> np.ndarray:
    """Concatenation over i of first[i], first[i] + 1, ..., first[i] + count[i] - 1 (int64; count >= 0), computed as
    one cumulative sum: a step array of ones whose entry at each run's start holds the jump from the previous run's
    last value (from 0 for the first run)."""
    total = int(count.sum())
    steps = np.ones(total, dtype=np.int64) if out is None else out
    if out is not None:
        steps[:] = 1
    keep = count > 0
    f, c = first[keep], count[keep]
    if f.size:
        starts = np.cumsum(c) - c
        prev_last = np.empty_like(f)
        prev_last[0] = 0
        prev_last[1:] = f[:-1] + c[:-1] - 1
        steps[starts] = f - prev_last
        np.cumsum(steps, out=steps)
    return steps


@dataclass
class _Batch:
    """Per-sequence integer columns of a step, and its block tables concatenated without padding."""

    length: np.ndarray      # int64 [n]
    cached: np.ndarray      # int64 [n]
    nblk: np.ndarray        # int64 [n], table entries per sequence
    flat: np.ndarray        # int64 [sum nblk], every table, back to back
    row_start: np.ndarray   # int64 [n], where each table starts in ``flat``

    @classmethod
    def of(cls, seqs) -> "_Batch":
        n = len(seqs)
        cols = np.array([(s.seq_length, s.num_cached_tokens, len(s.block_table)) for s in seqs],
                        dtype=np.int64).reshape(n, 3)
        nblk = cols[:, 2].copy()
        flat = np.fromiter((b for s in seqs for b in s.block_table), dtype=np.int64, count=int(nblk.sum()))
        row_start = np.zeros(n, dtype=np.int64)
        if n > 1:
            np.cumsum(nblk[:-1], out=row_start[1:])
        return cls(cols[:, 0].copy(), cols[:, 1].copy(), nblk, flat, row_start)

    def padded_tables(self, out: np.ndarray) -> None:
        """Writes the -1 padded [n, width] tables into ``out`` (rows in order, entries in order)."""
        out[...] = -1
        width = out.shape[1]
        if width and self.flat.size:
            out[np.arange(width)[None, :] < self.nblk[:, None]] = self.flat


def prefill_slots(batch: _Batch, block_size: int) -> np.ndarray:
    """Cache slot of every uncached token of every sequence that has a block table, in token order. A sequence's
    tokens [cached, length) touch blocks cached // bs .. (length - 1) // bs; inside each block their slots are
    consecutive, so each (sequence, block) piece is one run starting at table[block] * bs + first token % bs."""
    bs = block_size
    q = batch.length - batch.cached
    live = (q > 0) & (batch.nblk > 0)
    first_blk = np.where(live, batch.cached // bs, 0)
    pieces = np.where(live, (batch.length - 1) // bs - first_blk + 1, 0)
    col = _runs(first_blk, pieces)                                      # table column of each piece
    entry = batch.flat[_runs(batch.row_start + first_blk, pieces)]      # its block id
    lo = np.maximum(np.repeat(batch.cached, pieces), col * bs)          # first token of the piece
    hi = np.minimum(np.repeat(batch.length, pieces), (col + 1) * bs)    # one past its last token
    return _runs(entry * bs + lo - col * bs, hi - lo)


def prepare_prefill_context(seqs, block_size: int, device="cuda", graphs: bool = False,
                            staging: StepStaging | None = None) -> torch.Tensor:
    """Sets the prefill context of ``seqs`` and returns the positions of their uncached tokens (int64, on
    ``device``). Block tables are included when some sequence has a cached prefix or ``graphs`` is set (the
    prefill graphs read every key through the tables) (reference: nanovllm_voxcpm/engine/model_runner.py:851-911)."""
    batch = _Batch.of(seqs)
    n = len(seqs)
    q = batch.length - batch.cached
    total_q = int(q.sum())
    with_tables = graphs or bool((batch.cached > 0).any())
    slots = prefill_slots(batch, block_size)
    width = int(batch.nblk.max(initial=0))
    stage = staging or StepStaging(device)
    specs = [(np.int64, (total_q,)), (np.int32, (n + 1,)), (np.int32, (n + 1,)), (np.int32, (slots.size,))]
    if with_tables:
        specs.append((np.int32, (n, width)))
    views = stage.layout(specs)
    _runs(batch.cached, q, out=views[0])
    for cu, lens in ((views[1], q), (views[2], batch.length)):
        cu[0] = 0
        np.cumsum(lens, out=cu[1:])
    views[3][:] = slots
    if with_tables:
        batch.padded_tables(views[4])
    dev = stage.upload()
    set_context(True, dev[1], dev[2], int(q.max(initial=0)), int(batch.length.max(initial=0)), dev[3], None,
                dev[4] if with_tables else None)
    return dev[0]


def prepare_decode_context(seqs, block_size: int, device="cuda", staging: StepStaging | None = None
                           ) -> torch.Tensor:
    """Sets the decode context of ``seqs`` (one new token each, at position length - 1, stored in the table's last
    block) and returns the positions (reference: nanovllm_voxcpm/engine/model_runner.py:913-938)."""
    batch = _Batch.of(seqs)
    n = len(seqs)
    if (batch.nblk == 0).any():
        raise ValueError("decode: every sequence needs a block for its new token")
    width = int(batch.nblk.max(initial=0))
    stage = staging or StepStaging(device)
    pos, slot, lens, tables = stage.layout([(np.int64, (n,)), (np.int32, (n,)), (np.int32, (n,)),
                                            (np.int32, (n, width))])
    np.subtract(batch.length, 1, out=pos)
    last_entry = batch.flat[batch.row_start + batch.nblk - 1]
    slot[:] = last_entry * block_size + pos % block_size
    lens[:] = batch.length
    batch.padded_tables(tables)
    dev = stage.upload()
    set_context(False, slot_mapping=dev[1], context_lens=dev[2], block_tables=dev[3])
    return dev[0]


# ----------------------------------------------------------------------------------------------------------------------
# KV cache and decode graph buffers


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
