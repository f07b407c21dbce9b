"""The attention operators the reference's Attention.forward calls, on the gfx950 kernels of libvoxattn.so.

Names, argument meanings, shapes and returned layouts follow the calls the reference makes
(reference: nanovllm_voxcpm/model/layers.py:290-305 store_kvcache, :337-348 flash_attn_varlen_func,
:350-358 flash_attn_with_kvcache, :361 flash_attn_func). Every op runs on torch's current stream, allocates its
outputs with torch (graph-pool safe), never synchronizes, and raises when libvoxattn.so is missing: there is no
CPU or PyTorch fallback.

Supported shapes are the model's: head_dim 128, bf16 activations and caches (any 2-byte dtype for the KV store),
int32 index tensors. Decode takes up to 16 query heads over 1 or 2 KV heads.
"""

from __future__ import annotations

import threading

import torch

from . import _lib

HEAD_DIM = 128
MAX_DECODE_HEADS = 16


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise AssertionError(msg)


def _check_cuda(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t is not None and (t.device.type != "cuda" or t.device != dev):
            raise ValueError(f"all tensors must be on the same GPU, got {t.device} and {dev}")
    return dev


def _as_i32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype == torch.int32:
        return t if t.is_contiguous() else t.contiguous()
    if t.dtype in (torch.int64, torch.int16, torch.uint8, torch.int8):
        return t.to(torch.int32).contiguous()
    raise TypeError(f"{name} must be an integer tensor, got {t.dtype}")


# --------------------------------------------------------------------------------------------------------------------
# KV store


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    """Writes key[i] / value[i] ([N, HK, head_dim], token rows may be strided) to the cache slot slot_mapping[i];
    slot -1 is skipped. Caches are [num_blocks, block_size, HK, head_dim] (or any view whose slot rows are
    HK * head_dim apart). Bit-exact. Reference: nanovllm_voxcpm/model/layers.py:290-305 (same asserts)."""
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    _require(key.stride(-1) == 1 and value.stride(-1) == 1, "key/value: last dim must be contiguous")
    _require(key.stride(1) == head_dim and value.stride(1) == head_dim, "key/value: heads must be head_dim apart")
    _require(k_cache.stride(1) == D and v_cache.stride(1) == D, "caches: slot rows must be num_kv_heads*head_dim apart")
    _require(slot_mapping.numel() == N, "slot_mapping must hold one slot per token")
    if N == 0:
        return
    dev = _check_cuda(key, value, k_cache, v_cache, slot_mapping)
    if key.dtype != k_cache.dtype or value.dtype != v_cache.dtype or key.element_size() != 2:
        raise TypeError(f"store_kvcache: 16-bit key/value matching the cache dtype, got {key.dtype}/{k_cache.dtype}")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("store_kvcache: caches must be contiguous [num_blocks, block_size, HK, head_dim]")
    if k_cache.shape != v_cache.shape:
        raise ValueError(f"store_kvcache: k_cache {tuple(k_cache.shape)} and v_cache {tuple(v_cache.shape)} differ")
    slots = _as_i32(slot_mapping.reshape(-1), "slot_mapping")
    lib = _lib.load()
    _lib.check(lib.vox_store_kvcache(key.data_ptr(), value.data_ptr(), key.stride(0), value.stride(0),
                                     k_cache.data_ptr(), v_cache.data_ptr(), k_cache.numel() // D, slots.data_ptr(),
                                     N, num_heads, head_dim, _lib.stream_handle(dev)),
               "store_kvcache")


# --------------------------------------------------------------------------------------------------------------------
# Decode workspace and plans
#
# A decode call that reuses a plan reads the plan records and the step layout an earlier call left in the workspace, so
# the workspace is made once per device and workgroup count (room for a full 512-sequence launch; its layout depends on
# the workgroup count) and kept for the life of the process, since a captured graph holds its address. Decode calls on
# one device therefore share it and must not overlap (the engine runs them on one stream).
#
# Plans: the layout of a decode step (which tiles each workgroup walks) is the same for every layer of the step.
# Callers that know when a step's layout repeats pass a `plan` key (Attention.forward: the forward context, see
# layers.py); the first call with a new key records the layout in the workspace, later calls with the same key reuse
# it. The key also carries the graph capture in progress, so a capture always records its own plan in its first call.

_WS_LOCK = threading.Lock()
_WORKSPACE: dict[tuple[int, int], torch.Tensor] = {}
_PLANNED: dict[int, object] = {}


def _device_index(dev: torch.device) -> int:
    return dev.index if dev.index is not None else torch.cuda.current_device()


def decode_workspace(dev: torch.device) -> torch.Tensor:
    """The persistent decode workspace (uint8) of the device at the current workgroup count, made zero-filled on
    first use."""
    lib = _lib.load()
    key = (_device_index(dev), int(lib.vox_decode_workgroups()))
    with _WS_LOCK:
        ws = _WORKSPACE.get(key)
        if ws is None:
            ws = torch.zeros(max(int(lib.vox_decode_workspace_bytes(512)), 256), dtype=torch.uint8, device=dev)
            _WORKSPACE[key] = ws
        return ws


def _plan_mode(dev: torch.device, plan, *shape) -> int:
    """The plan mode of a call with key `plan` (None: no plan) over launch shape `shape` on `dev`'s workspace."""
    if plan is None:
        return _lib.PLAN_NONE
    lib = _lib.load()
    key = (plan, shape, int(lib.vox_decode_workgroups()), _lib.capture_id(_lib.stream_handle(dev)))
    idx = _device_index(dev)
    with _WS_LOCK:
        if _PLANNED.get(idx) == key:
            return _lib.PLAN_REUSE
        _PLANNED[idx] = key
        return _lib.PLAN_RECORD


_SCOPE = threading.local()


class planning:
    """Within the block, varlen calls made without a `plan` key use `key` (how Attention.forward plans the decode rows
    of a mixed step through flash_attn_varlen_func, whose signature is flash-attn's)."""

    def __init__(self, key):
        self.key = key

    def __enter__(self):
        self.prev = getattr(_SCOPE, "key", None)
        _SCOPE.key = self.key
        return self

    def __exit__(self, *exc):
        _SCOPE.key = self.prev
        return False


def forget_plans() -> None:
    """Drops every recorded plan key (the next planned call on each device records again)."""
    with _WS_LOCK:
        _PLANNED.clear()


# --------------------------------------------------------------------------------------------------------------------
# Decode


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, context_lens: torch.Tensor,
                     block_tables: torch.Tensor, softmax_scale: float, out: torch.Tensor | None = None,
                     key: torch.Tensor | None = None, value: torch.Tensor | None = None,
                     slot_mapping: torch.Tensor | None = None, plan=None) -> torch.Tensor:
    """One query token per sequence: q [B, H, 128] (sequence rows may be strided) over the paged cache
    [num_blocks, block_size, HK, 128] through block_tables int32 [B, max_blocks]; context_lens int32 [B].
    Returns o [B, H, 128] bf16 (contiguous). Rows with context_lens == 0 get zeros.

    With key / value ([B, HK, 128], rows may be strided) and slot_mapping ([B]), the decode step's KV store happens
    in the same call: the result (and the caches afterwards) are those of store_kvcache(key, value, k_cache,
    v_cache, slot_mapping) followed by this attention, as long as no sequence's slot lies inside another
    sequence's context (the engine's decode steps: each sequence writes its own last block).

    ``plan``: a hashable key that stays the same exactly as long as context_lens, block_tables and slot_mapping hold
    the same values (Attention.forward passes one per forward context): the first call with a key records the
    decode layout, later ones reuse it (see the plan notes above)."""
    B, H, D = q.shape
    dev = _check_cuda(q, k_cache, v_cache, context_lens, block_tables)
    if q.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise TypeError("decode attention takes bf16 q and caches")
    if D != HEAD_DIM or q.stride(2) != 1 or q.stride(1) != D:
        raise ValueError(f"q must be [B, H, {HEAD_DIM}] with contiguous heads, got {tuple(q.shape)} {q.stride()}")
    if k_cache.dim() != 4 or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous [num_blocks, block_size, HK, head_dim]")
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache shapes differ")
    num_blocks, block_size, HK, Dk = k_cache.shape
    if Dk != D:
        raise ValueError("cache head_dim differs from q's")
    if H % HK or H > MAX_DECODE_HEADS or HK not in (1, 2):
        raise ValueError(f"decode supports H <= {MAX_DECODE_HEADS} query heads over 1 or 2 KV heads, got {H}/{HK}")
    if context_lens.numel() != B or block_tables.dim() != 2 or block_tables.shape[0] < B:
        raise ValueError("context_lens must be [B] and block_tables [B, max_blocks]")
    if out is None:
        out = torch.empty(B, H, D, dtype=q.dtype, device=dev)
    if B == 0:
        return out
    if q.stride(0) == 0:
        q = q.contiguous()
    bt = block_tables if (block_tables.dtype == torch.int32 and block_tables.stride(1) == 1) else \
        _as_i32(block_tables, "block_tables")
    lens = _as_i32(context_lens.reshape(-1), "context_lens")
    max_blocks = bt.shape[1]
    lib = _lib.load()
    ws = decode_workspace(dev)
    mode = _plan_mode(dev, plan, "decode", key is not None, B, max_blocks, bt.stride(0), H, HK, block_size)
    if key is None:
        _lib.check(lib.vox_decode_attn(q.data_ptr(), q.stride(0), k_cache.data_ptr(), v_cache.data_ptr(), num_blocks,
                                       block_size, bt.data_ptr(), bt.stride(0), max_blocks, lens.data_ptr(), B, H, HK,
                                       D, float(softmax_scale), mode, ws.data_ptr(), ws.numel(), out.data_ptr(),
                                       _lib.stream_handle(dev)),
                   "decode_attn")
        return out
    _check_cuda(q, key, value, slot_mapping)
    if key.dtype != k_cache.dtype or value.dtype != v_cache.dtype:
        raise TypeError(f"decode store: key/value dtype {key.dtype}/{value.dtype} differs from the caches'")
    if key.shape != (B, HK, D) or value.shape != (B, HK, D):
        raise ValueError(f"decode store: key and value must be [{B}, {HK}, {D}], got {tuple(key.shape)}")
    if key.stride(2) != 1 or key.stride(1) != D or value.stride(2) != 1 or value.stride(1) != D:
        raise ValueError("decode store: key/value heads must be contiguous")
    if slot_mapping.numel() != B:
        raise ValueError("decode store: slot_mapping must hold one slot per sequence")
    slots = _as_i32(slot_mapping.reshape(-1), "slot_mapping")
    _lib.check(lib.vox_decode_attn_store(q.data_ptr(), q.stride(0), key.data_ptr(), value.data_ptr(), key.stride(0),
                                         value.stride(0), slots.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                         num_blocks, block_size, bt.data_ptr(), bt.stride(0), max_blocks,
                                         lens.data_ptr(), B, H, HK, D, float(softmax_scale), mode, ws.data_ptr(),
                                         ws.numel(), out.data_ptr(), _lib.stream_handle(dev)),
               "decode_attn_store")
    return out


# --------------------------------------------------------------------------------------------------------------------
# Prefill / varlen


def varlen_attention(q: torch.Tensor, k: torch.Tensor | None, v: torch.Tensor | None, *,
                     cu_seqlens_q: torch.Tensor | None, cu_seqlens_k: torch.Tensor | None, max_seqlen_q: int,
                     softmax_scale: float, causal: bool, block_table: torch.Tensor | None = None,
                     k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
                     batch: int | None = None, uniform_seqlen_q: int = 0, uniform_seqlen_k: int = 0,
                     out: torch.Tensor | None = None, quant: bool = False, inv_smooth: torch.Tensor | None = None,
                     plan=None):
    """The varlen prefill kernel. q [T, H, 128] (token rows may be strided). K/V from packed rows k / v
    [Tk, HK, 128] or, with block_table, from k_cache / v_cache [num_blocks, block_size, HK, 128]. Sequences from
    cu_seqlens_q / cu_seqlens_k (int32 [B + 1]) or, when both are None, `batch` sequences of uniform lengths.
    Returns o [T, H, 128] bf16; with ``quant`` (HK <= 2), (int8 o [T, H * 128], fp32 scale [T]): per token
    o * inv_smooth (fp32 [H * 128], optional) over all heads quantized to rint(o / scale), scale = max(amax, 1e-6) / 127
    (reference: the QUANT epilogues of kernels/prefill_attn.py:84-92, kernels/short_attn.py:55-64, 137-146).
    ``plan``: as decode_attention's, for the one-query rows a paged varlen call runs on the decode kernel."""
    T, H, D = q.shape
    dev = _check_cuda(q)
    if q.dtype != torch.bfloat16:
        raise TypeError("varlen attention takes bf16 q")
    if D != HEAD_DIM or q.stride(2) != 1 or q.stride(1) != D:
        raise ValueError(f"q must be [T, H, {HEAD_DIM}] with contiguous heads, got {tuple(q.shape)} {q.stride()}")
    if quant:
        out_q = torch.empty(T, H * D, dtype=torch.int8, device=dev)
        out_scale = torch.empty(T, dtype=torch.float32, device=dev)
        if inv_smooth is not None:
            _check_cuda(q, inv_smooth)
            if inv_smooth.numel() != H * D:
                raise ValueError(f"inv_smooth must hold H * head_dim = {H * D} values")
            inv_smooth = inv_smooth.reshape(-1).to(torch.float32).contiguous()
        out = (out_q, out_scale)
    elif out is None:
        out = torch.empty(T, H, D, dtype=q.dtype, device=dev)
    if cu_seqlens_q is not None:
        B = cu_seqlens_q.numel() - 1
        if cu_seqlens_k is None or cu_seqlens_k.numel() != B + 1:
            raise ValueError("cu_seqlens_k must have as many entries as cu_seqlens_q")
        cu_q = _as_i32(cu_seqlens_q, "cu_seqlens_q")
        cu_k = _as_i32(cu_seqlens_k, "cu_seqlens_k")
        _check_cuda(q, cu_q, cu_k)
    else:
        B = int(batch or 0)
        cu_q = cu_k = None
    if T == 0 or B <= 0 or max_seqlen_q <= 0:
        return out
    lib = _lib.load()
    if block_table is not None:
        if k_cache is None or v_cache is None:
            raise ValueError("block_table given without caches")
        _check_cuda(q, k_cache, v_cache, block_table)
        if k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
            raise TypeError("caches must be bf16")
        if k_cache.dim() != 4 or not (k_cache.is_contiguous() and v_cache.is_contiguous()) \
                or k_cache.shape != v_cache.shape or k_cache.shape[3] != D:
            raise ValueError("caches must be contiguous [num_blocks, block_size, HK, head_dim]")
        num_blocks, block_size, HK, _ = k_cache.shape
        bt = block_table if (block_table.dtype == torch.int32 and block_table.stride(1) == 1) else \
            _as_i32(block_table, "block_table")
        if bt.dim() != 2 or bt.shape[0] < B:
            raise ValueError("block_table must be [B, max_blocks]")
        args = (0, 0, 0, 0, k_cache.data_ptr(), v_cache.data_ptr(), num_blocks, block_size, bt.data_ptr(),
                bt.stride(0), bt.shape[1])
    else:
        if k is None or v is None:
            raise ValueError("packed K/V required without a block table")
        _check_cuda(q, k, v)
        if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
            raise TypeError("k/v must be bf16")
        HK = k.shape[1]
        if k.dim() != 3 or k.shape[2] != D or k.stride(2) != 1 or k.stride(1) != D or v.shape != k.shape \
                or v.stride(2) != 1 or v.stride(1) != D:
            raise ValueError("k/v must be [Tk, HK, head_dim] with contiguous heads")
        args = (k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0), 0, 0, 0, 0, 0, 0, 0)
    if H % HK:
        raise ValueError(f"num_heads {H} is not a multiple of num_kv_heads {HK}")
    if quant:
        # long sequences whose work items outnumber the CUs run as two passes (bf16 attention into a scratch buffer,
        # then the per-token quantization): the library sizes the scratch, 0 where the fused epilogue is faster
        ws_bytes = lib.vox_prefill_int8_workspace_bytes(T, B, int(max_seqlen_q), H, HK, D, 1 if causal else 0)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
        _lib.check(lib.vox_prefill_attn_int8(q.data_ptr(), q.stride(0), *args,
                                             None if cu_q is None else cu_q.data_ptr(),
                                             None if cu_k is None else cu_k.data_ptr(), B, int(max_seqlen_q),
                                             int(uniform_seqlen_q), int(uniform_seqlen_k), H, HK, D,
                                             float(softmax_scale), 1 if causal else 0,
                                             None if inv_smooth is None else inv_smooth.data_ptr(),
                                             out_q.data_ptr(), out_q.stride(0), out_scale.data_ptr(), T,
                                             None if ws is None else ws.data_ptr(), ws_bytes,
                                             _lib.stream_handle(dev)),
                   "prefill_attn_int8")
        return out
    # Paged varlen with one-query rows (the decode rows of a mixed prefill + decode step): those rows run on the
    # split-KV decode kernels and the rest on a persistent prefill grid, which the library does when it gets the
    # workspace. Passed when every row has one query, or when the (q tile, sequence) grid would be mostly empty
    # (T rows against B sequences of up to max_seqlen_q), which is what a few prefills beside many decode rows look
    # like; a dense prefill keeps the plain grid (a 44 x 46 paged step: 12.8 us there, 20.5 us persistent).
    ws, mode = None, _lib.PLAN_NONE
    if block_table is not None and cu_q is not None and (max_seqlen_q == 1 or 4 * T <= B * max_seqlen_q):
        ws = decode_workspace(dev)
        if plan is None:
            plan = getattr(_SCOPE, "key", None)
        mode = _plan_mode(dev, plan, "varlen", B, int(block_table.shape[1]), H, HK, int(k_cache.shape[1]))
    _lib.check(lib.vox_prefill_attn(q.data_ptr(), q.stride(0), *args,
                                    None if cu_q is None else cu_q.data_ptr(),
                                    None if cu_k is None else cu_k.data_ptr(), B, int(max_seqlen_q),
                                    int(uniform_seqlen_q), int(uniform_seqlen_k), H, HK, D, float(softmax_scale),
                                    1 if causal else 0, out.data_ptr(), out.stride(0), mode,
                                    None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
                                    _lib.stream_handle(dev)),
               "prefill_attn")
    return out


def prefill_attention_store(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                            v_cache: torch.Tensor, slot_mapping: torch.Tensor, *, cu_seqlens_q: torch.Tensor,
                            cu_seqlens_k: torch.Tensor, max_seqlen_q: int, softmax_scale: float, causal: bool = True,
                            out: torch.Tensor | None = None, block_table: torch.Tensor | None = None,
                            plan=None, quant: bool = False, inv_smooth: torch.Tensor | None = None):
    """store_kvcache(k, v, k_cache, v_cache, slot_mapping) then the varlen attention, as one call. Without a block
    table the attention reads the packed rows k / v (vox_prefill_attn_store: the copy rides in the attention launch).
    With one it reads the caches through the table (vox_prefill_attn_store_paged): a mixed step's launch takes each
    sequence's new keys from the rows and its merge kernel writes the caches; that needs slot_mapping to hold the
    slots the table gives the new tokens' positions, as the engine's does. Same outputs and caches as the two calls.
    ``plan``: as varlen_attention's (keys of its own, apart from varlen_attention's). ``quant``: the int8 output of
    varlen_attention(quant=True), (int8 o [T, H * D], fp32 scale [T]), with the copy riding in that launch
    (vox_prefill_attn_int8_store: the W8A8 layer's store_kvcache + short_causal_attention pair without a block table,
    its store_kvcache + paged_prefill_attention pair with one, nanovllm_voxcpm/kernels/fused_layer.py:619-667).
    Reference: the prefill branch of nanovllm_voxcpm/model/layers.py:326-348."""
    T, H, D = q.shape
    N, HK, Dk = k.shape
    _require(k.stride(-1) == 1 and v.stride(-1) == 1, "key/value: last dim must be contiguous")
    _require(k.stride(1) == Dk and v.stride(1) == Dk, "key/value: heads must be head_dim apart")
    _require(k_cache.stride(1) == HK * Dk and v_cache.stride(1) == HK * Dk,
             "caches: slot rows must be num_kv_heads*head_dim apart")
    _require(slot_mapping.numel() == N, "slot_mapping must hold one slot per token")
    dev = _check_cuda(q, k, v, k_cache, v_cache, slot_mapping, cu_seqlens_q, cu_seqlens_k)
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16 \
            or k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise TypeError("prefill_attention_store takes bf16 q, k, v and caches")
    if D != HEAD_DIM or Dk != HEAD_DIM or q.stride(2) != 1 or q.stride(1) != D or v.shape != k.shape:
        raise ValueError(f"q / k / v must be [T, H, {HEAD_DIM}] / [N, HK, {HEAD_DIM}] with contiguous heads")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()) or k_cache.shape != v_cache.shape:
        raise ValueError("caches must be contiguous [num_blocks, block_size, HK, head_dim] of one shape")
    if H % HK:
        raise ValueError(f"num_heads {H} is not a multiple of num_kv_heads {HK}")
    B = cu_seqlens_q.numel() - 1
    if cu_seqlens_k.numel() != B + 1:
        raise ValueError("cu_seqlens_k must have as many entries as cu_seqlens_q")
    cu_q = _as_i32(cu_seqlens_q, "cu_seqlens_q")
    cu_k = _as_i32(cu_seqlens_k, "cu_seqlens_k")
    slots = _as_i32(slot_mapping.reshape(-1), "slot_mapping")
    lib = _lib.load()
    bt = None
    if block_table is not None:
        _check_cuda(q, block_table)
        if k_cache.dim() != 4 or k_cache.shape[2] != HK:
            raise ValueError("with a block table the caches must be [num_blocks, block_size, HK, head_dim]")
        bt = block_table if (block_table.dtype == torch.int32 and block_table.stride(1) == 1) else \
            _as_i32(block_table, "block_table")
        if bt.dim() != 2 or bt.shape[0] < B:
            raise ValueError("block_table must be [B, max_blocks]")
    # the cache as [num_blocks, block_size] slots (a flat [slots, HK, D] cache: one slot per block)
    num_blocks, block_size = (k_cache.shape[0], k_cache.shape[1]) if k_cache.dim() == 4 else \
        (k_cache.numel() // (HK * Dk), 1)
    if quant:
        out_q = torch.empty(T, H * D, dtype=torch.int8, device=dev)
        out_scale = torch.empty(T, dtype=torch.float32, device=dev)
        if inv_smooth is not None:
            _check_cuda(q, inv_smooth)
            if inv_smooth.numel() != H * D:
                raise ValueError(f"inv_smooth must hold H * head_dim = {H * D} values")
            inv_smooth = inv_smooth.reshape(-1).to(torch.float32).contiguous()
        ws_bytes = lib.vox_prefill_int8_workspace_bytes(T, max(B, 0), int(max_seqlen_q), H, HK, D, 1 if causal else 0)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
        _lib.check(lib.vox_prefill_attn_int8_store(
            q.data_ptr(), q.stride(0), k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0), slots.data_ptr(), N,
            k_cache.data_ptr(), v_cache.data_ptr(), num_blocks, block_size, None if bt is None else bt.data_ptr(),
            0 if bt is None else bt.stride(0), 0 if bt is None else bt.shape[1], cu_q.data_ptr(), cu_k.data_ptr(),
            max(B, 0), int(max_seqlen_q) if T else 0, H, HK, D, float(softmax_scale), 1 if causal else 0,
            None if inv_smooth is None else inv_smooth.data_ptr(), out_q.data_ptr(), out_q.stride(0),
            out_scale.data_ptr(), T, None if ws is None else ws.data_ptr(), ws_bytes, _lib.stream_handle(dev)),
            "prefill_attn_int8_store")
        return out_q, out_scale
    if out is None:
        out = torch.empty(T, H, D, dtype=q.dtype, device=dev)
    if bt is not None:
        # the mixed launch (and with it the riding store) where varlen_attention would run the one-query rows on the
        # decode kernels
        ws, mode = None, _lib.PLAN_NONE
        if T and B > 0 and (max_seqlen_q == 1 or 4 * T <= B * max_seqlen_q):
            ws = decode_workspace(dev)
            if plan is None:
                plan = getattr(_SCOPE, "key", None)
            mode = _plan_mode(dev, plan, "varlen-store", B, int(bt.shape[1]), H, HK, int(block_size))
        _lib.check(lib.vox_prefill_attn_store_paged(
            q.data_ptr(), q.stride(0), k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0), slots.data_ptr(), N,
            k_cache.data_ptr(), v_cache.data_ptr(), num_blocks, block_size, bt.data_ptr(), bt.stride(0), bt.shape[1],
            cu_q.data_ptr(), cu_k.data_ptr(), max(B, 0), int(max_seqlen_q) if T else 0, H, HK, D, float(softmax_scale),
            1 if causal else 0, out.data_ptr(), out.stride(0), mode, None if ws is None else ws.data_ptr(),
            0 if ws is None else ws.numel(), _lib.stream_handle(dev)), "prefill_attn_store_paged")
        return out
    _lib.check(lib.vox_prefill_attn_store(q.data_ptr(), q.stride(0), k.data_ptr(), v.data_ptr(), k.stride(0),
                                          v.stride(0), slots.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                          k_cache.numel() // (HK * Dk), N, cu_q.data_ptr(), cu_k.data_ptr(), max(B, 0),
                                          int(max_seqlen_q) if T else 0, H, HK, D, float(softmax_scale),
                                          1 if causal else 0, out.data_ptr(), out.stride(0), _lib.stream_handle(dev)),
               "prefill_attn_store")
    return out


# --------------------------------------------------------------------------------------------------------------------
# The flash-attn entry points the reference's Attention.forward calls
#
# Same names, parameter order and defaults as flash-attn 2.8.3 (the version the reference pins: setup.sh:14,
# Dockerfile:37), so positional and keyword callers both bind as they do against flash-attn. Options this path
# does not implement (dropout, sliding windows, softcapping, ALiBi, returning probabilities or the LSE, appending new
# keys in flash_attn_with_kvcache) raise NotImplementedError when set to anything but their inactive default.


def _unsupported(fn: str, **opts) -> None:
    """Raises for any flash-attn option given a value other than its inactive default."""
    inactive = {"dropout_p": 0.0, "window_size": (-1, -1), "softcap": 0.0, "alibi_slopes": None,
                "return_attn_probs": False, "k": None, "v": None, "rotary_cos": None, "rotary_sin": None,
                "cache_batch_idx": None, "cache_leftpad": None, "return_softmax_lse": False}
    for name, value in opts.items():
        want = inactive[name]
        same = value is None if want is None else (tuple(value) == want if isinstance(want, tuple) else value == want)
        if not same:
            raise NotImplementedError(f"{fn}: {name}={value!r} is not supported (only {want!r})")


def flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, dropout_p=0.0,
                           softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0, alibi_slopes=None,
                           deterministic=False, return_attn_probs=False, block_table=None):
    """q [T, H, D]; k / v packed [Tk, HK, D], or the paged caches [num_blocks, block_size, HK, D] with
    block_table [B, max_blocks]. Returns o [T, H, D]. The kernel is deterministic whatever ``deterministic`` says.
    (Reference call: nanovllm_voxcpm/model/layers.py:337-348.)"""
    _unsupported("flash_attn_varlen_func", dropout_p=dropout_p, window_size=window_size, softcap=softcap,
                 alibi_slopes=alibi_slopes, return_attn_probs=return_attn_probs)
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    if block_table is not None:
        return varlen_attention(q, None, None, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k,
                                max_seqlen_q=max_seqlen_q, softmax_scale=scale, causal=causal,
                                block_table=block_table, k_cache=k, v_cache=v)
    return varlen_attention(q, k, v, cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_seqlens_k, max_seqlen_q=max_seqlen_q,
                            softmax_scale=scale, causal=causal)


def flash_attn_with_kvcache(q, k_cache, v_cache, k=None, v=None, rotary_cos=None, rotary_sin=None,
                            cache_seqlens=None, cache_batch_idx=None, cache_leftpad=None, block_table=None,
                            softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                            rotary_interleaved=True, alibi_slopes=None, num_splits=0, return_softmax_lse=False):
    """q [B, Lq, H, D] over the paged caches; cache_seqlens (int32 [B], or one int for every sequence) counts every
    key; returns o [B, Lq, H, D]. Lq == 1 (the engine's decode) runs the split-KV decode kernel, which picks its
    own split (``num_splits`` is not used); Lq > 1 runs the varlen kernel with bottom-right causal alignment.
    (Reference call: nanovllm_voxcpm/model/layers.py:350-358.)"""
    _unsupported("flash_attn_with_kvcache", k=k, v=v, rotary_cos=rotary_cos, rotary_sin=rotary_sin,
                 cache_batch_idx=cache_batch_idx, cache_leftpad=cache_leftpad, window_size=window_size,
                 softcap=softcap, alibi_slopes=alibi_slopes, return_softmax_lse=return_softmax_lse)
    if block_table is None or cache_seqlens is None:
        raise NotImplementedError("flash_attn_with_kvcache: the paged form (block_table, cache_seqlens) is supported")
    B, Lq, H, D = q.shape
    if isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((B,), cache_seqlens, dtype=torch.int32, device=q.device)
    scale = D ** -0.5 if softmax_scale is None else softmax_scale
    if Lq == 1:
        return decode_attention(q[:, 0], k_cache, v_cache, cache_seqlens, block_table, scale).unsqueeze(1)
    lens = _as_i32(cache_seqlens.reshape(-1), "cache_seqlens")
    cu_q = torch.arange(0, (B + 1) * Lq, Lq, dtype=torch.int32, device=q.device)
    cu_k = torch.zeros(B + 1, dtype=torch.int32, device=q.device)
    torch.cumsum(lens, 0, out=cu_k[1:])
    q3 = q.reshape(B * Lq, H, D)
    o = varlen_attention(q3, None, None, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=Lq,
                         softmax_scale=scale, causal=causal, block_table=block_table, k_cache=k_cache,
                         v_cache=v_cache)
    return o.view(B, Lq, H, D)


def _token_rows(x: torch.Tensor) -> torch.Tensor:
    """[B, L, heads, D] as [B*L, heads, D] token rows without a copy when rows are uniformly strided."""
    B, L, Hx, D = x.shape
    row = x.stride(1) if L > 1 else x.stride(0)
    if B > 1 and x.stride(0) != L * row:
        x = x.contiguous()
        row = Hx * D
    return x.as_strided((B * L, Hx, D), (row, x.stride(2), x.stride(3)))


def flash_attn_func(q, k, v, dropout_p=0.0, softmax_scale=None, causal=False, window_size=(-1, -1), softcap=0.0,
                    alibi_slopes=None, deterministic=False, return_attn_probs=False):
    """Dense attention q [B, L, H, D], k / v [B, Lk, HK, D] (the non-causal branch of Attention.forward: LocEnc and
    LocDiT rows). Returns o [B, L, H, D]. (Reference call: nanovllm_voxcpm/model/layers.py:359-361.)"""
    _unsupported("flash_attn_func", dropout_p=dropout_p, window_size=window_size, softcap=softcap,
                 alibi_slopes=alibi_slopes, return_attn_probs=return_attn_probs)
    B, L, H, D = q.shape
    Lk = k.shape[1]
    scale = D ** -0.5 if softmax_scale is None else softmax_scale
    o = varlen_attention(_token_rows(q), _token_rows(k), _token_rows(v), cu_seqlens_q=None, cu_seqlens_k=None,
                         max_seqlen_q=L, softmax_scale=scale, causal=causal, batch=B, uniform_seqlen_q=L,
                         uniform_seqlen_k=Lk)
    return o.view(B, L, H, D)
