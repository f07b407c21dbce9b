"""GPU parity of the KV slot scatter (HIP kernel 1) against the oracle: bit-exact."""

from __future__ import annotations

import pytest
import torch

from oracle import attention as ref
from tests._util import BLOCK, D, HK, paged_pool, randn
from voxcpm2_arabic_dialects_turbo_amd.ops import store_kvcache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_kv_store_writes_each_token_to_its_slot():
    """The reference's known-answer case (tests/test_kernel_references.py:240-257)."""
    gen = torch.Generator().manual_seed(3)
    k_cache = torch.zeros(4, BLOCK, HK, D, device=DEV, dtype=torch.bfloat16)
    v_cache = torch.zeros_like(k_cache)
    k, v = randn(gen, 9, HK, D).to(DEV), randn(gen, 9, HK, D).to(DEV)
    slots = torch.tensor([5, 300, 511, 512, 1023, -1, 0, 700, 256], device=DEV, dtype=torch.int32)
    store_kvcache(k, v, k_cache, v_cache, slots)
    torch.cuda.synchronize()
    flat_k, flat_v = k_cache.view(-1, HK, D), v_cache.view(-1, HK, D)
    for i, slot in enumerate(slots.tolist()):
        if slot >= 0:
            assert torch.equal(flat_k[slot], k[i]) and torch.equal(flat_v[slot], v[i]), i
    assert int((flat_k.abs().sum((1, 2)) > 0).sum()) == 8  # nothing else written


def _qkv_views(gen, n):
    """q / k / v as views of one [n, (16 + 2 + 2) * 128] qkv output, as the model's split produces them."""
    qkv = randn(gen, n, (16 + 2 * HK) * D).to(DEV)
    q, k, v = qkv.split([16 * D, HK * D, HK * D], dim=-1)
    return qkv, q.view(n, 16, D), k.view(n, HK, D), v.view(n, HK, D)


def test_store_config2_shape_strided_rows_bit_exact():
    """benchmark config 2: ~2304 prefill tokens of 8 sequences scattered into 256-token blocks of a 512-block pool."""
    gen = torch.Generator().manual_seed(20)
    lens = torch.randint(64, 513, (8,), generator=gen).tolist()
    _, _, tables = paged_pool(gen, lens, 512)
    slots = torch.cat([torch.tensor([ref.slot_of(tables[b].tolist(), j, BLOCK) for j in range(n)])
                       for b, n in enumerate(lens)]).to(torch.int32)
    _, _, k, v = _qkv_views(gen, len(slots))
    assert k.stride(0) == (16 + 2 * HK) * D
    k_cache = torch.zeros(512, BLOCK, HK, D, device=DEV, dtype=torch.bfloat16)
    v_cache = torch.zeros_like(k_cache)
    store_kvcache(k, v, k_cache, v_cache, slots.to(DEV))
    want_k, want_v = torch.zeros(512, BLOCK, HK, D, dtype=torch.bfloat16), torch.zeros(512, BLOCK, HK, D,
                                                                                      dtype=torch.bfloat16)
    ref.store_kvcache(k.cpu(), v.cpu(), want_k, want_v, slots)
    assert torch.equal(k_cache.cpu(), want_k) and torch.equal(v_cache.cpu(), want_v)


def test_store_unaligned_rows_take_the_element_path():
    """Rows that are not 16-byte aligned (odd element offset) are still copied exactly."""
    gen = torch.Generator().manual_seed(21)
    base = randn(gen, 40 * 2 * HK * D + 1).to(DEV)
    k = base[1:1 + 40 * HK * D].view(40, HK, D)
    v = base[1 + 40 * HK * D:1 + 80 * HK * D].view(40, HK, D)
    assert k.data_ptr() % 16 != 0
    slots = torch.randperm(4 * BLOCK, generator=gen)[:40].to(torch.int32)
    k_cache = torch.zeros(4, BLOCK, HK, D, device=DEV, dtype=torch.bfloat16)
    v_cache = torch.zeros_like(k_cache)
    store_kvcache(k, v, k_cache, v_cache, slots.to(DEV))
    want_k, want_v = torch.zeros(4, BLOCK, HK, D, dtype=torch.bfloat16), torch.zeros(4, BLOCK, HK, D,
                                                                                    dtype=torch.bfloat16)
    ref.store_kvcache(k.cpu(), v.cpu(), want_k, want_v, slots)
    assert torch.equal(k_cache.cpu(), want_k) and torch.equal(v_cache.cpu(), want_v)


def test_store_skips_padding_and_out_of_range_slots_and_takes_int64():
    gen = torch.Generator().manual_seed(22)
    k, v = randn(gen, 6, HK, D).to(DEV), randn(gen, 6, HK, D).to(DEV)
    k_cache = torch.zeros(2, BLOCK, HK, D, device=DEV, dtype=torch.bfloat16)
    v_cache = torch.zeros_like(k_cache)
    slots = torch.tensor([3, -1, 2 * BLOCK, 511, 2 * BLOCK + 7, 0], dtype=torch.int64)
    store_kvcache(k, v, k_cache, v_cache, slots.to(DEV))
    flat = k_cache.view(-1, HK, D).cpu()
    assert torch.equal(flat[3], k[0].cpu()) and torch.equal(flat[511], k[3].cpu()) and torch.equal(flat[0], k[5].cpu())
    assert int((flat.float().abs().sum((1, 2)) > 0).sum()) == 3


def test_store_of_zero_tokens_is_a_no_op():
    k_cache = torch.zeros(1, BLOCK, HK, D, device=DEV, dtype=torch.bfloat16)
    e = torch.zeros(0, HK, D, device=DEV, dtype=torch.bfloat16)
    store_kvcache(e, e, k_cache, k_cache, torch.zeros(0, device=DEV, dtype=torch.int32))
    assert int(k_cache.abs().sum()) == 0
