"""Seeded random configurations of the decode and varlen prefill kernels against the oracle (max-abs 2e-2,
mean-abs 2e-3): batch sizes, ragged and empty lengths, cached prefixes, block sizes, head groupings, split grids,
causal and non-causal, packed and paged keys drawn together, so that combinations the targeted tests do not name are
exercised too. Each case is small enough for the oracle's per-sequence loop."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as ref
from tests._util import D, attn_close, paged_pool, randn
from voxcpm2_arabic_dialects_turbo_amd import _lib
from voxcpm2_arabic_dialects_turbo_amd.ops import decode_attention, flash_attn_varlen_func

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = D ** -0.5


def _cu(lens):
    return torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32)


@pytest.mark.parametrize("seed", range(12))
def test_random_decode_configurations(seed):
    gen = torch.Generator().manual_seed(1000 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=gen))]
    h, hk = pick([(16, 2), (8, 1), (16, 1), (4, 2)])
    bs = pick([32, 64, 256])  # the decode ABI takes block sizes that are multiples of 32
    B = int(torch.randint(1, 300, (1,), generator=gen))
    lens = []
    for _ in range(B):
        u = float(torch.rand(1, generator=gen))
        lens.append(0 if u < 0.15 else int(torch.randint(1, 200 if u < 0.5 else 3000, (1,), generator=gen)))
    pool = sum((max(n, 1) + bs - 1) // bs for n in lens) + 2
    kc, vc, tables = paged_pool(gen, [max(n, 1) for n in lens], pool, block_size=bs, hk=hk)
    q = randn(gen, B, h, D)
    grid = pick([0, 0, 5, 100])
    lib = _lib.load()
    lib.vox_set_decode_workgroups(grid)
    try:
        out = decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV),
                               tables.to(DEV), SCALE)
        torch.cuda.synchronize()
    finally:
        lib.vox_set_decode_workgroups(0)
    want = ref.decode(q.float(), kc, vc, lens, tables, SCALE)
    attn_close(out, want, f"seed {seed}: B={B} heads {h}/{hk} block {bs} grid {grid}")


@pytest.mark.parametrize("seed", range(12))
def test_random_varlen_prefill_configurations(seed):
    gen = torch.Generator().manual_seed(2000 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=gen))]
    h, hk = pick([(16, 2), (8, 1), (16, 4), (16, 16)])
    paged = bool(torch.randint(2, (1,), generator=gen))
    causal = bool(torch.randint(4, (1,), generator=gen))  # causal three times in four
    B = int(torch.randint(1, 12, (1,), generator=gen))
    nq = [int(torch.randint(1, 300, (1,), generator=gen)) for _ in range(B)]
    if paged:
        bs = pick([32, 64, 256])
        nk = [n + (int(torch.randint(0, 600, (1,), generator=gen)) if causal else 0) for n in nq]
        pool = sum((n + bs - 1) // bs for n in nk) + 2
        kc, vc, tables = paged_pool(gen, nk, pool, block_size=bs, hk=hk)
    else:
        nk = list(nq)
        k, v = randn(gen, sum(nk), hk, D), randn(gen, sum(nk), hk, D)
    q = randn(gen, sum(nq), h, D)
    cq, ck = _cu(nq), _cu(nk)
    if paged:
        out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), cq.to(DEV), ck.to(DEV), max(nq), max(nk),
                                     softmax_scale=SCALE, causal=causal, block_table=tables.to(DEV))
        want = ref.varlen(q.float(), cq, ck, scale=SCALE, causal=causal, k_cache=kc, v_cache=vc,
                          block_tables=tables)
    else:
        out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cq.to(DEV), ck.to(DEV), max(nq), max(nk),
                                     softmax_scale=SCALE, causal=causal)
        want = ref.varlen(q.float(), cq, ck, scale=SCALE, causal=causal, k=k, v=v)
    torch.cuda.synchronize()
    attn_close(out, want, f"seed {seed}: B={B} heads {h}/{hk} paged={paged} causal={causal}")


@pytest.mark.parametrize("seed", range(8))
def test_random_int8_prefill_configurations(seed):
    """The int8-output prefill (fused epilogue or, for long causal batches, the bf16 pass and the quantization
    pass) under the int8 tests' bounds, with or without inv_smooth."""
    from tests.test_prefill_int8_gpu import _check
    from voxcpm2_arabic_dialects_turbo_amd.ops import varlen_attention

    gen = torch.Generator().manual_seed(3000 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=gen))]
    h, hk = pick([(16, 2), (8, 1), (16, 1)])
    paged = bool(torch.randint(2, (1,), generator=gen))
    causal = bool(torch.randint(4, (1,), generator=gen))
    B = int(torch.randint(1, 11, (1,), generator=gen))
    nq = [int(torch.randint(1, 320, (1,), generator=gen)) for _ in range(B)]
    inv = torch.rand(h * D, generator=gen) + 0.5 if bool(torch.randint(2, (1,), generator=gen)) else None
    q = randn(gen, sum(nq), h, D)
    cq = _cu(nq)
    if paged:
        bs = pick([64, 256])
        nk = [n + (int(torch.randint(0, 400, (1,), generator=gen)) if causal else 0) for n in nq]
        kc, vc, tables = paged_pool(gen, nk, sum((n + bs - 1) // bs for n in nk) + 2, block_size=bs, hk=hk)
        ck = _cu(nk)
        out = varlen_attention(q.to(DEV), None, None, cu_seqlens_q=cq.to(DEV), cu_seqlens_k=ck.to(DEV),
                               max_seqlen_q=max(nq), softmax_scale=SCALE, causal=causal, block_table=tables.to(DEV),
                               k_cache=kc.to(DEV), v_cache=vc.to(DEV), quant=True,
                               inv_smooth=None if inv is None else inv.to(DEV))
        want = ref.varlen(q.float(), cq, ck, scale=SCALE, causal=causal, k_cache=kc, v_cache=vc,
                          block_tables=tables)
    else:
        k, v = randn(gen, sum(nq), hk, D), randn(gen, sum(nq), hk, D)
        out = varlen_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu_seqlens_q=cq.to(DEV), cu_seqlens_k=cq.to(DEV),
                               max_seqlen_q=max(nq), softmax_scale=SCALE, causal=causal, quant=True,
                               inv_smooth=None if inv is None else inv.to(DEV))
        want = ref.varlen(q.float(), cq, cq, scale=SCALE, causal=causal, k=k, v=v)
    torch.cuda.synchronize()
    _check(out, want, f"seed {seed}: B={B} heads {h}/{hk} paged={paged} causal={causal}", inv)


@pytest.mark.parametrize("seed", range(8))
def test_random_decode_with_the_store_configurations(seed):
    """The decode call with the step's store folded in (what Attention.forward runs for a decode step) against the
    oracle's store followed by its decode: outputs within the tolerance, caches bit-exact. The new token sits at each
    sequence's last position; padded rows (context 0, slot -1) among them; random grids."""
    gen = torch.Generator().manual_seed(4000 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=gen))]
    h, hk = pick([(16, 2), (8, 1)])
    bs = pick([32, 256])
    B = int(torch.randint(1, 200, (1,), generator=gen))
    lens = [0 if float(torch.rand(1, generator=gen)) < 0.1 else int(torch.randint(1, 2500, (1,), generator=gen))
            for _ in range(B)]
    kc, vc, tables = paged_pool(gen, [max(n, 1) for n in lens], sum(-(-max(n, 1) // bs) for n in lens) + 2,
                                block_size=bs, hk=hk)
    q, key, value = randn(gen, B, h, D), randn(gen, B, hk, D), randn(gen, B, hk, D)
    slots = torch.tensor([-1 if n == 0 else int(tables[b, (n - 1) // bs]) * bs + (n - 1) % bs
                          for b, n in enumerate(lens)], dtype=torch.int32)
    k_ref, v_ref = kc.clone(), vc.clone()
    ref.store_kvcache(key, value, k_ref, v_ref, slots)
    want = ref.decode(q.float(), k_ref, v_ref, lens, tables, SCALE)
    grid = pick([0, 7, 300])
    lib = _lib.load()
    lib.vox_set_decode_workgroups(grid)
    try:
        k1, v1 = kc.to(DEV), vc.to(DEV)
        out = decode_attention(q.to(DEV), k1, v1, torch.tensor(lens, dtype=torch.int32, device=DEV), tables.to(DEV),
                               SCALE, key=key.to(DEV), value=value.to(DEV), slot_mapping=slots.to(DEV))
        torch.cuda.synchronize()
    finally:
        lib.vox_set_decode_workgroups(0)
    attn_close(out, want, f"seed {seed}: B={B} heads {h}/{hk} block {bs} grid {grid}")
    assert torch.equal(k1.cpu(), k_ref) and torch.equal(v1.cpu(), v_ref), f"seed {seed}: caches differ"


@pytest.mark.parametrize("seed", range(10))
def test_random_prefill_with_the_store_configurations(seed):
    """Prefill calls with the step's store riding in them through the block tables (prefill_attention_store, what
    Attention.forward runs for a prefill or mixed step with caches) against the oracle's store followed by its varlen
    attention over the stored caches: outputs within the tolerance, caches bit-exact. Random prefixes (so the first
    new key falls anywhere in a tile), one-query rows among the prefills (the mixed launch when the grid is sparse,
    the plain forms otherwise), block sizes 64-512 (and 32: the two calls), head groupings 16/2 and 8/1, decode grids."""
    from voxcpm2_arabic_dialects_turbo_amd.ops import prefill_attention_store

    gen = torch.Generator().manual_seed(5000 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=gen))]
    h, hk = pick([(16, 2), (8, 1)])
    bs = pick([64, 128, 256, 512, 32])
    n_pre, n_dec = int(torch.randint(1, 8, (1,), generator=gen)), pick([0, 3, 40, 150])
    nq = [int(torch.randint(2, 300, (1,), generator=gen)) for _ in range(n_pre)] + [1] * n_dec
    prefix = [pick([0, 0, int(torch.randint(1, 700, (1,), generator=gen))]) for _ in range(n_pre)]
    nk = [a + b for a, b in zip(nq[:n_pre], prefix)] + [int(torch.randint(1, 2000, (1,), generator=gen))
                                                         for _ in range(n_dec)]
    order = torch.randperm(len(nq), generator=gen).tolist()  # prefills and one-query rows interleaved
    nq, nk = [nq[i] for i in order], [nk[i] for i in order]
    kc, vc, tables = paged_pool(gen, nk, sum(-(-n // bs) for n in nk) + 2, block_size=bs, hk=hk)
    T = sum(nq)
    q, key, value = randn(gen, T, h, D), randn(gen, T, hk, D), randn(gen, T, hk, D)
    slots = torch.tensor([ref.slot_of(tables[b].tolist(), j, bs) for b in range(len(nk))
                          for j in range(nk[b] - nq[b], nk[b])], dtype=torch.int32)
    k_ref, v_ref = kc.clone(), vc.clone()
    ref.store_kvcache(key, value, k_ref, v_ref, slots)
    want = ref.varlen(q.float(), _cu(nq), _cu(nk), k_cache=k_ref, v_cache=v_ref, block_tables=tables)
    grid = pick([0, 0, 7, 300])
    lib = _lib.load()
    lib.vox_set_decode_workgroups(grid)
    try:
        k1, v1 = kc.to(DEV), vc.to(DEV)
        out = prefill_attention_store(q.to(DEV), key.to(DEV), value.to(DEV), k1, v1, slots.to(DEV),
                                      cu_seqlens_q=_cu(nq).to(DEV), cu_seqlens_k=_cu(nk).to(DEV),
                                      max_seqlen_q=max(nq), softmax_scale=SCALE, block_table=tables.to(DEV))
        torch.cuda.synchronize()
    finally:
        lib.vox_set_decode_workgroups(0)
    what = f"seed {seed}: {n_pre} prefills + {n_dec} one-query rows, heads {h}/{hk}, block {bs}, grid {grid}"
    attn_close(out, want, what)
    assert torch.equal(k1.cpu(), k_ref) and torch.equal(v1.cpu(), v_ref), f"{what}: caches differ"
