"""CPU restatement of the attention path's math (test infrastructure only; see oracle/__init__.py).

All functions take and return CPU torch tensors and compute in the dtype of their inputs (callers upcast to fp32 as
the reference's tests do, or to fp64 for tight checks).
"""

from __future__ import annotations

import torch


def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, scale: float | None = None
           ) -> torch.Tensor:
    """Softmax attention of one sequence, GQA by repeat_interleave.

    q [n_q, H, D], k / v [n_k, HK, D]; with ``causal`` query i sees keys j <= n_k - n_q + i (bottom-right aligned).
    Returns [n_q, H * D]. Reference: tests/test_kernel_references.py:161-170 (``_attend``; the scale there is
    D ** -0.5, here a parameter that defaults to it)."""
    H, HK = q.shape[1], k.shape[1]
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    k, v = k.repeat_interleave(H // HK, 1), v.repeat_interleave(H // HK, 1)
    att = torch.einsum("qhd,khd->hqk", q, k) * scale
    if causal:
        n_q, n_k = q.shape[0], k.shape[0]
        mask = torch.arange(n_k)[None, :] > (n_k - n_q + torch.arange(n_q))[:, None]
        att = att.masked_fill(mask[None], float("-inf"))
    return torch.einsum("hqk,khd->qhd", att.softmax(-1), v).reshape(q.shape[0], -1)


def gather_pages(cache: torch.Tensor, table, n: int) -> torch.Tensor:
    """The first n tokens of one sequence's K or V through its block table: cache [pages, page, HK, D].
    Reference: tests/test_kernel_references.py:199-201 (``k_cache[pages].reshape(-1, HK, D)[:n_k]``); only the
    ceil(n / page) pages those tokens occupy are read, so padded or stale table columns are never touched."""
    page = cache.shape[1]
    pages = torch.as_tensor(table, dtype=torch.long)[:(n + page - 1) // page]
    HK, D = cache.shape[2], cache.shape[3]
    return cache[pages].reshape(-1, HK, D)[:n]


def slot_of(table, j: int, block_size: int) -> int:
    """Cache slot of token j: block_table[j // block_size] * block_size + j % block_size.
    Reference: nanovllm_voxcpm/engine/model_runner.py:883 (prefill), :919 (decode)."""
    return int(table[j // block_size]) * block_size + j % block_size


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping) -> None:
    """In place: k_cache.flat[slot * row : (slot + 1) * row] = key[i] for every slot != -1 (same for value), where
    row = HK * D. Reference: nanovllm_voxcpm/model/layers.py:266-287 (store_kvcache_kernel)."""
    row = key.shape[1] * key.shape[2]
    flat_k, flat_v = k_cache.view(-1, row), v_cache.view(-1, row)
    for i, slot in enumerate(torch.as_tensor(slot_mapping).tolist()):
        if slot == -1:
            continue
        flat_k[slot] = key[i].reshape(row)
        flat_v[slot] = value[i].reshape(row)


def decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, context_lens, block_tables,
           scale: float | None = None) -> torch.Tensor:
    """One query token per sequence over its first context_lens[b] cached tokens: q [B, H, D] -> [B, H, D].
    The decode call of Attention.forward (reference: nanovllm_voxcpm/model/layers.py:349-358), defined by
    ``attend`` over the page gather; a sequence with no context gives zeros (the HIP kernel's convention for padded
    rows; the reference leaves them unspecified)."""
    B, H, D = q.shape
    out = torch.zeros(B, H, D, dtype=q.dtype)
    lens = torch.as_tensor(context_lens).tolist()
    for b in range(B):
        n = int(lens[b])
        if n <= 0:
            continue
        k = gather_pages(k_cache, block_tables[b], n).to(q.dtype)
        v = gather_pages(v_cache, block_tables[b], n).to(q.dtype)
        out[b] = attend(q[b:b + 1], k, v, causal=True, scale=scale).view(H, D)
    return out


def varlen(q: torch.Tensor, cu_seqlens_q, cu_seqlens_k, scale: float | None = None, causal: bool = True,
           k: torch.Tensor | None = None, v: torch.Tensor | None = None, k_cache: torch.Tensor | None = None,
           v_cache: torch.Tensor | None = None, block_tables=None) -> torch.Tensor:
    """Varlen attention: q [T, H, D]; keys from packed k / v [Tk, HK, D] (rows cu_seqlens_k[b] ..) or, with
    block_tables, through the page gather. Returns [T, H, D]. The prefill call of Attention.forward
    (reference: nanovllm_voxcpm/model/layers.py:334-348; its paged test: tests/test_kernel_references.py:196-203)."""
    T, H, D = q.shape
    out = torch.zeros(T, H, D, dtype=q.dtype)
    cu_q = torch.as_tensor(cu_seqlens_q).tolist()
    cu_k = torch.as_tensor(cu_seqlens_k).tolist()
    for b in range(len(cu_q) - 1):
        q0, q1 = int(cu_q[b]), int(cu_q[b + 1])
        nk = int(cu_k[b + 1]) - int(cu_k[b])
        if q1 == q0:
            continue
        if block_tables is not None:
            kb = gather_pages(k_cache, block_tables[b], nk).to(q.dtype)
            vb = gather_pages(v_cache, block_tables[b], nk).to(q.dtype)
        else:
            kb = k[int(cu_k[b]):int(cu_k[b + 1])].to(q.dtype)
            vb = v[int(cu_k[b]):int(cu_k[b + 1])].to(q.dtype)
        out[q0:q1] = attend(q[q0:q1], kb, vb, causal=causal, scale=scale).view(q1 - q0, H, D)
    return out


def dense(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float | None = None, causal: bool = False
          ) -> torch.Tensor:
    """Batched attention q [B, L, H, D], k / v [B, Lk, HK, D] -> [B, L, H, D] (the non-causal branch,
    reference: nanovllm_voxcpm/model/layers.py:359-361; its test: tests/test_kernel_references.py:229-237)."""
    B, L, H, D = q.shape
    return torch.stack([attend(q[b], k[b], v[b], causal=causal, scale=scale).view(L, H, D) for b in range(B)])


def quantize_rows(x: torch.Tensor, inv_smooth: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row int8 quantization the W8A8 o_proj consumes: x [M, K] (fp32) -> (int8 [M, K], fp32 scale [M]) with
    y = x * inv_smooth, amax = max(max |y|, 1e-6), scale = amax / 127, q = rint(y / scale) (round half to even).
    Reference: nanovllm_voxcpm/kernels/int8_linear.py:19-30 (``_quant_rows``), the same epilogue as
    kernels/prefill_attn.py:84-92 and kernels/short_attn.py:55-64, 137-146 apply to the attention output."""
    y = x.float() if inv_smooth is None else x.float() * inv_smooth.float().reshape(1, -1)
    amax = y.abs().amax(dim=1).clamp_min(1e-6)
    scale = amax / 127.0
    q = torch.round(y / scale[:, None])  # torch.round rounds half to even, as rint
    return q.to(torch.int8), scale


def dequantize_rows(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """q * scale per row (reference: tests/test_kernel_references.py:162-163, ``_deq``)."""
    return q.float() * scale.float()[:, None]


def close(out: torch.Tensor, ref: torch.Tensor, rel: float) -> float:
    """max|out - ref| <= rel * max|ref| (reference: tests/test_kernel_references.py:51-55); returns the ratio."""
    err = (out.float() - ref.float()).abs().max().item()
    peak = ref.abs().max().item()
    assert err <= rel * peak, f"max error {err:.3g} > {rel} x {peak:.3g}"
    return err / peak if peak else 0.0
