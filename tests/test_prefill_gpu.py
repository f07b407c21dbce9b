"""GPU parity of the varlen prefill kernel (HIP kernel 2) against the oracle and the golden vectors:
max-abs <= 2e-2, mean-abs <= 2e-3, and the reference tests' own rel 0.02 bound on their cases."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import attention as ref
from tests._util import BLOCK, D, H, HK, attn_close, paged_pool, randn, uniform_lens
from tests.golden import make_golden
from voxcpm2_arabic_dialects_turbo_amd import _lib
from voxcpm2_arabic_dialects_turbo_amd.kernels.prefill_attn import paged_prefill_attention
from voxcpm2_arabic_dialects_turbo_amd.kernels.short_attn import short_attention, short_causal_attention
from voxcpm2_arabic_dialects_turbo_amd.ops import flash_attn_func, flash_attn_varlen_func, store_kvcache

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = D ** -0.5
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")


def _golden(name):
    return torch.from_numpy(np.load(GOLDEN, allow_pickle=False)[f"{name}__out"])


def _cu(lens):
    return torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32)


def test_paged_prefill_over_a_cached_prefix_reference_case():
    """tests/test_kernel_references.py:179-207: a sequence without prefix, one with 293 cached tokens, one
    single-token prefill after 260, through scattered 256-token pages."""
    inp = make_golden.inputs("paged_prefill")
    d = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    out = paged_prefill_attention(d["q"], d["k_cache"], d["v_cache"], d["tables"], d["cu_q"], d["cu_k"], 7, SCALE)
    assert out.shape == (13, H * D) and out.dtype == torch.bfloat16
    want = ref.varlen(inp["q"].float(), inp["cu_q"], inp["cu_k"], k_cache=inp["k_cache"], v_cache=inp["v_cache"],
                      block_tables=inp["tables"])
    ref.close(out.cpu(), want.view(13, -1), 0.02)
    attn_close(out.view(13, H, D), want, "paged prefill vs oracle")
    attn_close(out.view(13, H, D), _golden("paged_prefill"), "paged prefill vs golden")
    # the same through flash_attn_varlen_func (Attention.forward's call)
    out2 = flash_attn_varlen_func(d["q"], d["k_cache"], d["v_cache"], max_seqlen_q=7, cu_seqlens_q=d["cu_q"],
                                  max_seqlen_k=300, cu_seqlens_k=d["cu_k"], softmax_scale=SCALE, causal=True,
                                  block_table=d["tables"])
    assert torch.equal(out2.view(13, -1), out)


def test_short_causal_reference_case():
    """tests/test_kernel_references.py:210-228: packed lens [1, 7, 16, 32, 3], causal over their own tokens."""
    inp = make_golden.inputs("short_causal")
    out = short_causal_attention(inp["q"].to(DEV), inp["k"].to(DEV), inp["v"].to(DEV), inp["cu"].to(DEV), 32, SCALE)
    want = ref.varlen(inp["q"].float(), inp["cu"], inp["cu"], k=inp["k"], v=inp["v"])
    ref.close(out.cpu(), want.view(59, -1), 0.02)
    attn_close(out.view(59, H, D), want, "short causal")
    attn_close(out.view(59, H, D)[:, make_golden.STORED_HEADS], _golden("short_causal"), "short causal vs golden")


@pytest.mark.parametrize("L", [1, 5, 11, 16])
def test_non_causal_short_rows(L):
    """LocEnc / LocDiT rows (tests/test_kernel_references.py:229-237): B = 6 sequences of L tokens, non-causal."""
    gen = torch.Generator().manual_seed(40 + L)
    q, k, v = randn(gen, 6, L, H, D), randn(gen, 6, L, HK, D), randn(gen, 6, L, HK, D)
    want = ref.dense(q.float(), k.float(), v.float())
    out = short_attention(q.to(DEV), k.to(DEV), v.to(DEV), SCALE)
    attn_close(out.view(6, L, H, D), want, f"short_attention L={L}")
    out2 = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), softmax_scale=SCALE, causal=False)
    assert out2.shape == (6, L, H, D) and torch.equal(out2.reshape(6 * L, -1), out)


def test_dense_golden():
    inp = make_golden.inputs("dense")
    out = flash_attn_func(inp["q"].to(DEV), inp["k"].to(DEV), inp["v"].to(DEV), softmax_scale=SCALE)
    attn_close(out[:, :, make_golden.STORED_HEADS], _golden("dense"), "dense vs golden")


@pytest.mark.parametrize("mode", ["packed", "paged"])
def test_config2_store_then_prefill(mode):
    """benchmark config 2: 8 sequences of U[64, 512] tokens packed by cu_seqlens; K/V stored into 256-token blocks of
    a 512-block pool, then causal prefill over the step's own k / v (packed) or through the block tables (paged)."""
    gen = torch.Generator().manual_seed(50)
    lens = uniform_lens(gen, 8, 64, 512)
    T = sum(lens)
    kc, vc, tables = paged_pool(gen, lens, 512)
    qkv = randn(gen, T, (H + 2 * HK) * D).to(DEV)
    q, k, v = qkv.split([H * D, HK * D, HK * D], dim=-1)
    q, k, v = q.view(T, H, D), k.view(T, HK, D), v.view(T, HK, D)
    slots = torch.cat([torch.tensor([ref.slot_of(tables[b].tolist(), j, BLOCK) for j in range(n)])
                       for b, n in enumerate(lens)]).to(torch.int32)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    store_kvcache(k, v, kc_d, vc_d, slots.to(DEV))
    cu = _cu(lens).to(DEV)
    if mode == "packed":
        out = flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), softmax_scale=SCALE, causal=True)
    else:
        out = flash_attn_varlen_func(q, kc_d, vc_d, cu, cu, max(lens), max(lens), softmax_scale=SCALE, causal=True,
                                     block_table=tables.to(DEV))
    want = ref.varlen(q.float().cpu(), _cu(lens), _cu(lens), k=k.cpu(), v=v.cpu())
    attn_close(out, want, f"config 2 {mode}")


def test_config5_mixed_prefill_and_decode_rows():
    """benchmark config 5: one varlen paged call with 6 new prefills (U[300, 600] tokens, stored first) and 120 decode
    rows (one query over U[128, 1800] cached tokens), 2048-block pool."""
    gen = torch.Generator().manual_seed(51)
    pre = uniform_lens(gen, 6, 300, 600)
    dec = uniform_lens(gen, 120, 128, 1800)
    nk = pre + dec
    nq = pre + [1] * 120
    kc, vc, tables = paged_pool(gen, nk, 2048)
    Tq = sum(nq)
    q = randn(gen, Tq, H, D)
    k_new, v_new = randn(gen, sum(pre), HK, D), randn(gen, sum(pre), HK, D)
    slots = torch.cat([torch.tensor([ref.slot_of(tables[b].tolist(), j, BLOCK) for j in range(n)])
                       for b, n in enumerate(pre)]).to(torch.int32)
    kc_d, vc_d = kc.to(DEV), vc.to(DEV)
    store_kvcache(k_new.to(DEV), v_new.to(DEV), kc_d, vc_d, slots.to(DEV))
    ref.store_kvcache(k_new, v_new, kc, vc, slots)
    out = flash_attn_varlen_func(q.to(DEV), kc_d, vc_d, _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq), max(nk),
                                 softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
    want = ref.varlen(q.float(), _cu(nq), _cu(nk), k_cache=kc, v_cache=vc, block_tables=tables)
    attn_close(out, want, "config 5")


def test_last_rows_one_query_per_sequence_over_all_keys():
    """The residual LM's last layer (kernels/fused_layer.py:767-773): cu_seqlens_q = arange(n + 1), max_seqlen_q = 1,
    keys = every row of the step (packed, cu_seqlens_k)."""
    gen = torch.Generator().manual_seed(52)
    lens = [5, 33, 1, 200]
    T = sum(lens)
    k, v = randn(gen, T, HK, D), randn(gen, T, HK, D)
    q_last = randn(gen, len(lens), H, D)
    cu_q = torch.arange(len(lens) + 1, dtype=torch.int32)
    out = flash_attn_varlen_func(q_last.to(DEV), k.to(DEV), v.to(DEV), cu_q.to(DEV), _cu(lens).to(DEV), 1,
                                 max(lens), softmax_scale=SCALE, causal=True)
    want = ref.varlen(q_last.float(), cu_q, _cu(lens), k=k, v=v)
    attn_close(out, want, "last rows")


def test_zero_length_sequences_in_a_padded_batch():
    """A captured prefill bucket pads with zero-length sequences; they produce no rows and disturb nothing."""
    gen = torch.Generator().manual_seed(53)
    nq = [0, 17, 0, 0, 64, 0]
    nk = [0, 17, 0, 0, 300, 0]
    kc, vc, tables = paged_pool(gen, [max(n, 1) for n in nk], 16)
    q = randn(gen, sum(nq), H, D)
    out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(nq).to(DEV), _cu(nk).to(DEV), 64, 300,
                                 softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
    want = ref.varlen(q.float(), _cu(nq), _cu(nk), k_cache=kc, v_cache=vc, block_tables=tables)
    attn_close(out, want, "zero-length sequences")


@pytest.mark.parametrize("bs", [32, 64, 128, 512])
def test_paged_block_sizes(bs):
    """Both paged key paths: a block size that is a multiple of the 64-key tile (one block id per tile) and one
    that is not (32: one block id per 16-byte piece), over cached prefixes with ragged last tiles."""
    gen = torch.Generator().manual_seed(56 + bs)
    nq = [37, 1, 130, 64]
    nk = [37 + 90, 1 + 700, 130, 64 + 63]
    kc, vc, tables = paged_pool(gen, nk, sum((n + bs - 1) // bs for n in nk) + 3, block_size=bs)
    q = randn(gen, sum(nq), H, D)
    out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq),
                                 max(nk), softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
    want = ref.varlen(q.float(), _cu(nq), _cu(nk), k_cache=kc, v_cache=vc, block_tables=tables)
    attn_close(out, want, f"paged block_size {bs}")


@pytest.mark.parametrize("h,hk", [(16, 1), (8, 1), (16, 4), (4, 4), (16, 8), (64, 2), (64, 1), (128, 1)])
def test_group_sizes(h, hk):
    """Every group size that divides a workgroup's 128 rows: 1 to 16 query heads per kv head, and 32, 64 and 128,
    where a 16-row wave holds part of one token's heads and an item fewer tokens than waves (128: one token)."""
    gen = torch.Generator().manual_seed(54 + h + hk)
    lens = [1, 70, 129, 33]
    T = sum(lens)
    q, k, v = randn(gen, T, h, D), randn(gen, T, hk, D), randn(gen, T, hk, D)
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), _cu(lens).to(DEV), _cu(lens).to(DEV), max(lens),
                                 max(lens), softmax_scale=SCALE, causal=True)
    attn_close(out, ref.varlen(q.float(), _cu(lens), _cu(lens), k=k, v=v), f"H={h} HK={hk}")


@pytest.mark.parametrize("h,hk,paged", [(16, 2, False), (16, 2, True), (16, 1, False), (16, 4, True)])
def test_rank_major_grid_of_causal_items_beyond_two_per_cu(h, hk, paged):
    """Causal grids of 64-row work items that exceed two per CU (512 on an MI355X) but not four run rank-major, the
    heaviest q tile of every (sequence, kv head) first: group sizes 16, 8 and 4, packed and paged with cached
    prefixes (bottom-right aligned), sequences of very different lengths (the short ones' high ranks are empty)."""
    gen = torch.Generator().manual_seed(61 + h + hk + paged)
    nq = [200, 3, 500, 77, 300, 129] if hk < 4 else [600, 1, 310, 64]
    pre = [50, 0, 300, 10, 0, 1] if paged else [0] * len(nq)
    nk = [a + b for a, b in zip(nq, pre)]
    g = h // hk
    assert 512 < -(-max(nq) // (64 // g)) * len(nq) * hk <= 1024  # the rank-major form on a 256-CU part
    q = randn(gen, sum(nq), h, D)
    if paged:
        kc, vc, tables = paged_pool(gen, nk, sum(-(-n // BLOCK) for n in nk) + 2, hk=hk)
        out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq),
                                     max(nk), softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
        want = ref.varlen(q.float(), _cu(nq), _cu(nk), k_cache=kc, v_cache=vc, block_tables=tables)
    else:
        k, v = randn(gen, sum(nk), hk, D), randn(gen, sum(nk), hk, D)
        out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq),
                                     max(nk), softmax_scale=SCALE, causal=True)
        want = ref.varlen(q.float(), _cu(nq), _cu(nk), k=k, v=v)
    attn_close(out, want, f"rank-major H={h} HK={hk} paged={paged}")


def test_long_sequences_compute_bound_shape():
    """Longer sequences (the compute-bound prefill shape the bench also reports): 4 x U[1024, 2048] tokens."""
    gen = torch.Generator().manual_seed(55)
    lens = uniform_lens(gen, 4, 1024, 2048)
    T = sum(lens)
    q, k, v = randn(gen, T, H, D), randn(gen, T, HK, D), randn(gen, T, HK, D)
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), _cu(lens).to(DEV), _cu(lens).to(DEV), max(lens),
                                 max(lens), softmax_scale=SCALE, causal=True)
    attn_close(out, ref.varlen(q.float(), _cu(lens), _cu(lens), k=k, v=v), "long causal")


def test_prefill_closed_forms_identical_keys():
    """With every key of a sequence identical the causal softmax is uniform over the visible keys: query i of a
    packed sequence gets mean(V[0..i]); query 0 gets V[0] exactly (one visible key, p = 1)."""
    gen = torch.Generator().manual_seed(57)
    lens = [1, 70, 200]
    T = sum(lens)
    q, v = randn(gen, T, H, D), randn(gen, T, HK, D)
    k = randn(gen, 1, HK, D).expand(T, HK, D).contiguous()
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), _cu(lens).to(DEV), _cu(lens).to(DEV), max(lens),
                                 max(lens), softmax_scale=SCALE, causal=True).float().cpu()
    at = 0
    for n in lens:
        vs = v[at:at + n].float()
        want = (vs.cumsum(0) / torch.arange(1, n + 1).view(n, 1, 1)).repeat_interleave(H // HK, dim=1)
        got = out[at:at + n]
        assert torch.equal(got[0], vs[0].repeat_interleave(H // HK, dim=0)), "query 0 must return V[0] exactly"
        err = (got - want).abs().max().item()
        assert err <= 2e-2, f"sequence of {n}: max-abs {err}"
        at += n


def test_prefill_scores_growing_across_key_tiles():
    """Later key tiles score far above the first (log2-scaled scores hundreds of units higher), which sends those
    tiles down the recompute-with-their-max path of the softmax; the result still matches the oracle, with no
    overflow, for packed and paged keys."""
    gen = torch.Generator().manual_seed(58)
    L = 300
    u = torch.randn(HK, D, generator=gen)  # a direction per kv group; every query leans along its group's
    q = (u.repeat_interleave(H // HK, dim=0).expand(L, H, D) + 0.3 * torch.randn(L, H, D, generator=gen))
    q = q.to(torch.bfloat16)
    k = randn(gen, L, HK, D).float()
    v = randn(gen, L, HK, D)
    # keys 64.. point along u with growing magnitude: raw scores up to ~1500, each key tile ~50+ log2 units above
    # the last
    for j in range(64, L):
        k[j] = u * (0.05 * (j - 63))
    k = k.to(torch.bfloat16)
    cu = _cu([L])
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), cu.to(DEV), L, L, softmax_scale=SCALE,
                                 causal=True)
    want = ref.varlen(q.float(), cu, cu, k=k, v=v)
    assert torch.isfinite(out.float()).all()
    attn_close(out, want, "growing scores, packed")
    kc, vc, tables = paged_pool(gen, [L], 4)
    for j in range(L):
        kc[tables[0, j // BLOCK], j % BLOCK] = k[j]
        vc[tables[0, j // BLOCK], j % BLOCK] = v[j]
    out2 = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), cu.to(DEV), cu.to(DEV), L, L,
                                  softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
    attn_close(out2, want, "growing scores, paged")


@pytest.mark.parametrize("paged", [False, True])
def test_scores_growing_across_key_tiles_in_the_32_row_form(paged):
    """The same growing scores in a grid above 2048 workgroups (one 2100-token sequence beside seven short ones:
    132 q tiles x 8 x 2), which takes the 4-wave x 32-row form and its pipelined loop, where a tile whose scores
    pass the running max is redone at the start of the next step; about every second key tile of the long sequence
    takes that path."""
    gen = torch.Generator().manual_seed(59)
    lens = [2100] + [int(x) for x in torch.randint(20, 120, (7,), generator=gen)]
    T = sum(lens)
    u = torch.randn(HK, D, generator=gen)
    q = (u.repeat_interleave(H // HK, dim=0).expand(T, H, D) + 0.3 * torch.randn(T, H, D, generator=gen))
    q = q.to(torch.bfloat16)
    k = randn(gen, T, HK, D).float()
    v = randn(gen, T, HK, D)
    for j in range(64, lens[0]):
        k[j] = u * (0.05 * (j - 63))
    k = k.to(torch.bfloat16)
    cu = _cu(lens)
    want = ref.varlen(q.float(), cu, cu, k=k, v=v)
    if paged:
        kc, vc, tables = paged_pool(gen, lens, sum((n + BLOCK - 1) // BLOCK for n in lens) + 2)
        at = 0
        for b, n in enumerate(lens):
            for j in range(n):
                kc[tables[b, j // BLOCK], j % BLOCK] = k[at + j]
                vc[tables[b, j // BLOCK], j % BLOCK] = v[at + j]
            at += n
        out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), cu.to(DEV), cu.to(DEV), max(lens),
                                     max(lens), softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
    else:
        out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), cu.to(DEV), cu.to(DEV), max(lens), max(lens),
                                     softmax_scale=SCALE, causal=True)
    assert torch.isfinite(out.float()).all()
    attn_close(out, want, f"growing scores, 32-row form, paged={paged}")


def _without_columns(table, drop, width):
    """A block-table row without the given columns, -1 padded to ``width``."""
    kept = [int(x) for j, x in enumerate(table.tolist()) if j not in drop and x >= 0]
    return kept + [-1] * (width - len(kept))


@pytest.mark.parametrize("bs", [256, 32])
def test_paged_unmapped_blocks_are_masked_and_slots_past_the_keys_stay_unread(bs):
    """Block-table entries inside a sequence's context that address no block (-1, or past the pool) are masked:
    their keys take no weight, as in the decode kernel. Expected: the oracle over the same sequence with those
    blocks' keys removed (each such block lies wholly inside the cached prefix, before the first query's position,
    so every query would have seen all of its keys and the causal alignment of the others is unchanged); a sequence
    whose whole context is unmapped gives zeros. Cache slots past a sequence's keys hold NaN and are never used.
    256: the tiles that go straight to LDS (range-checked loads); 32: the register-staged per-piece path."""
    gen = torch.Generator().manual_seed(71 + bs)
    nq = [50, 3, 20]
    nk = [50 + 600, 3 + 300, 20 + 40]
    pool = sum((n + bs - 1) // bs for n in nk) + 2
    kc, vc, tables = paged_pool(gen, nk, pool, block_size=bs)
    for b, n in enumerate(nk):  # NaN in every slot past the sequence's keys
        for j in range((n + bs - 1) // bs):
            used = min(bs, n - j * bs)
            kc[tables[b, j], used:] = float("nan")
            vc[tables[b, j], used:] = float("nan")
    t_gpu = tables.clone()
    t_gpu[0, 1] = -1            # keys bs .. 2 bs - 1 of sequence 0 (inside its 600-token prefix)
    t_gpu[1, 0] = pool + 5      # keys 0 .. bs - 1 of sequence 1 (inside its 300-token prefix)
    whole = (nk[2] + bs - 1) // bs
    t_gpu[2, :whole] = -7       # every key of sequence 2
    q = randn(gen, sum(nq), H, D)
    out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq),
                                 max(nk), softmax_scale=SCALE, causal=True, block_table=t_gpu.to(DEV))
    assert torch.isfinite(out.float()).all()
    width = tables.shape[1]
    t_ref = torch.tensor([_without_columns(tables[0], {1}, width), _without_columns(tables[1], {0}, width)],
                         dtype=torch.int32)
    nk_ref = [nk[0] - bs, nk[1] - bs]
    want = ref.varlen(q[:nq[0] + nq[1]].float(), _cu(nq[:2]), _cu(nk_ref), k_cache=kc, v_cache=vc,
                      block_tables=t_ref)
    attn_close(out[:nq[0] + nq[1]], want, f"unmapped blocks masked, block_size {bs}")
    assert out[nq[0] + nq[1]:].float().abs().max().item() == 0.0, "a fully unmapped context gives zeros"


def test_large_ragged_grid_in_per_xcd_order():
    """A grid of 128 q tiles x 8 sequences x 2 kv heads (>= 1024 workgroups: the launcher deals contiguous work
    ranges per XCD) with ragged lengths, so most ranges mix empty and full q tiles; packed and paged keys."""
    gen = torch.Generator().manual_seed(74)
    lens = [2048, 100, 1500, 7, 900, 2047, 64, 1300]
    T = sum(lens)
    q, k, v = randn(gen, T, H, D), randn(gen, T, HK, D), randn(gen, T, HK, D)
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), _cu(lens).to(DEV), _cu(lens).to(DEV), max(lens),
                                 max(lens), softmax_scale=SCALE, causal=True)
    want = ref.varlen(q.float(), _cu(lens), _cu(lens), k=k, v=v)
    attn_close(out, want, "per-XCD order, packed")
    nq = [max(1, n // 3) for n in lens]  # new tokens over cached prefixes
    kc, vc, tables = paged_pool(gen, lens, sum((n + BLOCK - 1) // BLOCK for n in lens) + 4)
    qp = randn(gen, sum(nq), H, D)
    outp = flash_attn_varlen_func(qp.to(DEV), kc.to(DEV), vc.to(DEV), _cu(nq).to(DEV), _cu(lens).to(DEV), max(nq),
                                  max(lens), softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
    wantp = ref.varlen(qp.float(), _cu(nq), _cu(lens), k_cache=kc, v_cache=vc, block_tables=tables)
    attn_close(outp, wantp, "per-XCD order, paged")


@pytest.mark.parametrize("causal", [False, True])
def test_uniform_lengths_over_several_key_tiles(causal):
    """The uniform-length mode (no cu_seqlens: flash_attn_func) over several 64-key tiles with a ragged last one:
    3 sequences of 300 queries over 333 keys, non-causal and bottom-right causal."""
    gen = torch.Generator().manual_seed(76 + causal)
    B, L, Lk = 3, 300, 333
    q, k, v = randn(gen, B, L, H, D), randn(gen, B, Lk, HK, D), randn(gen, B, Lk, HK, D)
    out = flash_attn_func(q.to(DEV), k.to(DEV), v.to(DEV), softmax_scale=SCALE, causal=causal)
    want = ref.dense(q.float(), k.float(), v.float(), causal=causal)
    attn_close(out, want, f"uniform lengths, causal={causal}")


def test_paged_table_wider_than_64_columns():
    """Block ids of the first 64 table columns come from the row held across the wave's lanes; a longer row (here
    64-token blocks under a 4930-key prefix: 78 columns) reads the columns past 63 from memory. Queries at the end
    of the long sequence walk tiles on both sides of column 64."""
    gen = torch.Generator().manual_seed(57)
    nq = [30, 5]
    nk = [4930, 70]
    kc, vc, tables = paged_pool(gen, nk, sum((n + 63) // 64 for n in nk) + 3, block_size=64)
    assert tables.shape[1] > 64
    q = randn(gen, sum(nq), H, D)
    out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq),
                                 max(nk), softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
    want = ref.varlen(q.float(), _cu(nq), _cu(nk), k_cache=kc, v_cache=vc, block_tables=tables)
    attn_close(out, want, "paged table of 78 columns")


@pytest.mark.parametrize("bs", [None, 256, 48])
def test_grid_above_the_eight_wave_limit(bs):
    """A grid of more than 2048 workgroups (128 q tiles x 12 sequences x 2 kv heads), which the launcher runs with
    4-wave workgroups of 32 rows each (smaller grids take 8 waves of 16 rows): one 2048-token causal sequence among
    short ones, packed keys and paged caches (block size 256: one block id per key tile; 48: per-piece block ids)."""
    gen = torch.Generator().manual_seed(81 + (bs or 0))
    lens = [2048, 50, 7, 300, 1, 129, 64, 77, 1000, 3, 250, 16]
    T = sum(lens)
    q = randn(gen, T, H, D)
    if bs is None:
        k, v = randn(gen, T, HK, D), randn(gen, T, HK, D)
        out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), _cu(lens).to(DEV), _cu(lens).to(DEV), max(lens),
                                     max(lens), softmax_scale=SCALE, causal=True)
        want = ref.varlen(q.float(), _cu(lens), _cu(lens), k=k, v=v)
    else:
        kc, vc, tables = paged_pool(gen, lens, sum((n + bs - 1) // bs for n in lens) + 2, block_size=bs)
        out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(lens).to(DEV), _cu(lens).to(DEV), max(lens),
                                     max(lens), softmax_scale=SCALE, causal=True,
                                     block_table=tables.to(DEV))
        want = ref.varlen(q.float(), _cu(lens), _cu(lens), k_cache=kc, v_cache=vc, block_tables=tables)
    attn_close(out, want, f"4-wave grid, block_size {bs}")


@pytest.mark.parametrize("bs", [256, 32])
def test_paged_gather_is_bit_exact_where_a_query_sees_one_key(bs):
    """Paged prefill without a prefix, through a shuffled block table: query 0 of every sequence sees only key 0, so
    its output is that key's V row exactly (p = 1), bit for bit, wherever the table put the block. 256: tiles straight
    to LDS; 32: the per-piece path."""
    gen = torch.Generator().manual_seed(80 + bs)
    lens = [1, 64, 300, 33, 257]
    pool = sum((n + bs - 1) // bs for n in lens) + 5
    kc, vc, tables = paged_pool(gen, lens, pool, block_size=bs)
    q = randn(gen, sum(lens), H, D)
    out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(lens).to(DEV), _cu(lens).to(DEV), max(lens),
                                 max(lens), softmax_scale=SCALE, causal=True, block_table=tables.to(DEV)).cpu()
    at = 0
    for b, n in enumerate(lens):
        v0 = vc[int(tables[b, 0]), 0]  # [HK, D]: key 0 of sequence b
        assert torch.equal(out[at], v0.repeat_interleave(H // HK, dim=0)), f"sequence {b}: query 0 != V[key 0]"
        at += n


def test_varlen_one_query_rows_run_on_the_decode_kernels():
    """A paged varlen call whose one-query sequences go to the split-KV decode kernels while the prefill kernel takes
    the rest: 600 sequences (two decode launches of up to 512), mixing zero-query padding, one-query rows (one of
    them with no keys, which gives zeros), and multi-query rows with and without a cached prefix; 64-token blocks."""
    gen = torch.Generator().manual_seed(90)
    nq, nk = [], []
    for i in range(600):
        kind = i % 6
        q_ = [0, 1, 1, 1, 5, 37][kind]
        k_ = 0 if kind == 0 else (q_ + int(torch.randint(0, 200, (1,), generator=gen)) if kind != 5 else q_)
        if i == 7:
            k_ = 0  # a one-query row with no keys
        nq.append(q_)
        nk.append(k_)
    bs = 64
    pool = sum((n + bs - 1) // bs for n in nk) + 3
    kc, vc, tables = paged_pool(gen, nk, pool, block_size=bs)
    q = randn(gen, sum(nq), H, D)
    out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq),
                                 max(nk), softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
    want = ref.varlen(q.float(), _cu(nq), _cu(nk), k_cache=kc, v_cache=vc, block_tables=tables)
    attn_close(out, want, "one-query rows on the decode kernels")
    row7 = sum(nq[:7])
    assert out[row7].float().abs().max().item() == 0.0, "a one-query row without keys gives zeros"


def test_mixed_step_captured_in_a_hip_graph_replays_like_eager():
    """A mixed prefill + decode varlen call runs on the caller's stream: one launch whose prefill workgroups take the
    multi-query rows and whose decode workgroups take the one-query rows, then the decode merge kernel. Captured in a
    HIP graph and replayed four times, with eager calls on other inputs between the replays, every replay equals the
    eager result bit for bit, which is within tolerance of the oracle."""
    gen = torch.Generator().manual_seed(91)
    pre, dec = [300, 450, 77], [700, 130, 1500, 2, 999]
    nk, nq = pre + dec, pre + [1] * len(dec)
    kc, vc, tables = paged_pool(gen, nk, 40)
    q = randn(gen, sum(nq), H, D)
    q2 = randn(gen, sum(nq), H, D)
    d = dict(k=kc.to(DEV), v=vc.to(DEV), cu_seqlens_q=_cu(nq).to(DEV), cu_seqlens_k=_cu(nk).to(DEV),
             max_seqlen_q=max(nq), max_seqlen_k=max(nk), softmax_scale=SCALE, causal=True,
             block_table=tables.to(DEV))
    q_d, q2_d = q.to(DEV), q2.to(DEV)
    eager = flash_attn_varlen_func(q_d, **d)
    eager2 = flash_attn_varlen_func(q2_d, **d)
    torch.cuda.synchronize()
    attn_close(eager, ref.varlen(q.float(), _cu(nq), _cu(nk), k_cache=kc, v_cache=vc, block_tables=tables), "eager")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static = flash_attn_varlen_func(q_d, **d)
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, eager), f"replay {r} differs from the eager call"
        other = flash_attn_varlen_func(q2_d, **d)
        torch.cuda.synchronize()
        assert torch.equal(other, eager2)


@pytest.mark.parametrize("n,bs", [(4200, 32), (8500, BLOCK)])
def test_mixed_step_with_a_prefill_longer_than_the_rank_order_covers(n, bs):
    """A mixed step (one-query rows on the decode kernels) whose prefill spans more than 1024 query tiles takes the
    persistent prefill's sequence-by-sequence order: 16 query heads over 1 kv head, a prefill of n tokens beside ten
    decode rows; with 32-token blocks the persistent prefill launch (4 tokens per tile) then the decode launch, with
    256-token blocks the mixed launch (8 tokens per tile). Its first and last 100 query rows are checked against the
    oracle."""
    gen = torch.Generator().manual_seed(92)
    H1, HK1 = 16, 1
    dec = [300, 77, 1, 256, 257, 900, 5, 600, 1000, 2]
    nq, nk = [n] + [1] * len(dec), [n] + dec
    width = (n + bs - 1) // bs
    pool = width + sum((x + bs - 1) // bs for x in dec) + 2
    kc = randn(gen, pool, bs, HK1, D)
    vc = randn(gen, pool, bs, HK1, D)
    perm = torch.randperm(pool, generator=gen).tolist()
    tables = torch.full((len(nk), width), -1, dtype=torch.int32)
    at = 0
    for b, x in enumerate(nk):
        nb = (x + bs - 1) // bs
        tables[b, :nb] = torch.tensor(perm[at:at + nb])
        at += nb
    q = randn(gen, sum(nq), H1, D)
    out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq),
                                 max(nk), softmax_scale=SCALE, causal=True, block_table=tables.to(DEV)).cpu()
    k0 = ref.gather_pages(kc, tables[0], n).float()
    v0 = ref.gather_pages(vc, tables[0], n).float()
    for i0, i1 in ((0, 100), (n - 100, n)):
        want = ref.attend(q[i0:i1].float(), k0[:i1], v0[:i1], causal=True, scale=SCALE).view(i1 - i0, H1, D)
        attn_close(out[i0:i1], want, f"long prefill rows {i0}:{i1}")
    want = ref.varlen(q[n:].float(), _cu(nq[1:]), _cu(nk[1:]), k_cache=kc, v_cache=vc, block_tables=tables[1:])
    attn_close(out[n:], want, "decode rows beside the long prefill")


def _mixed_case(gen, n_dec, dec_hi, pre_lens, hk, block_size=64):
    """A mixed step: prefills pre_lens (with a cached prefix of up to 100 tokens) and n_dec one-query rows over
    0..dec_hi keys, a paged pool of block_size-token blocks with hk kv heads."""
    nq = list(pre_lens) + [1] * n_dec
    nk = [n + int(torch.randint(0, 101, (1,), generator=gen)) for n in pre_lens] + \
        torch.randint(0, dec_hi + 1, (n_dec,), generator=gen).tolist()
    pool = sum((n + block_size - 1) // block_size for n in nk) + 5
    kc, vc, tables = paged_pool(gen, nk, pool, block_size=block_size, hk=hk)
    return nq, nk, kc, vc, tables


@pytest.mark.parametrize("grid", [1, 8, 0])
@pytest.mark.parametrize("h,hk", [(16, 2), (16, 1)])
def test_mixed_launch_with_many_decode_rows_per_workgroup(grid, h, hk):
    """The mixed launch (one-query rows on decode workgroups, each sharing a CU with a prefill workgroup, rounds of
    three sequences with bf16 wave partials): 248 one-query rows over 0-40 keys and 8 prefills (256 sequences, the
    launch's limit), over a decode grid of 1, 8 or one workgroup per CU, so that one workgroup's range holds from a
    few to every row (one round to a hundred)."""
    gen = torch.Generator().manual_seed(93 + grid + hk)
    nq, nk, kc, vc, tables = _mixed_case(gen, 248, 40, uniform_lens(gen, 8, 2, 200), hk)
    q = randn(gen, sum(nq), h, D)
    lib = _lib.load()
    lib.vox_set_decode_workgroups(grid)
    try:
        out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq),
                                     max(nk), softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
        torch.cuda.synchronize()
    finally:
        lib.vox_set_decode_workgroups(0)
    want = ref.varlen(q.float(), _cu(nq), _cu(nk), k_cache=kc, v_cache=vc, block_tables=tables)
    attn_close(out, want, f"mixed launch, decode grid {grid}, {h}/{hk} heads")
    zero_rows = [sum(nq[:b]) for b in range(8, 256) if nk[b] == 0]
    for r in zero_rows:
        assert out[r].float().abs().max().item() == 0.0, "a one-query row without keys gives zeros"


@pytest.mark.parametrize("h,hk", [(2, 2), (4, 2), (8, 2), (2, 1), (4, 1)])
def test_mixed_launch_group_sizes(h, hk):
    """The mixed launch at group sizes 1, 2 and 4 (the decode role's block-diagonal query columns mostly padding):
    40 one-query rows over up to 1500 keys (sequences cut across decode workgroups, merged by the merge kernel) beside
    5 prefills with cached prefixes, at the default decode grid."""
    gen = torch.Generator().manual_seed(96 + 3 * h + hk)
    nq, nk, kc, vc, tables = _mixed_case(gen, 40, 1500, uniform_lens(gen, 5, 2, 300), hk, block_size=BLOCK)
    q = randn(gen, sum(nq), h, D)
    out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq),
                                 max(nk), softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
    torch.cuda.synchronize()
    want = ref.varlen(q.float(), _cu(nq), _cu(nk), k_cache=kc, v_cache=vc, block_tables=tables)
    attn_close(out, want, f"mixed launch, {h}/{hk} heads")


@pytest.mark.parametrize("n_seq", [256, 257])
def test_mixed_step_at_and_past_the_mixed_launch_limit(n_seq):
    """256 sequences run as one mixed launch, 257 as the persistent prefill launch then the decode launch: both
    against the oracle (config-5 lengths: prefills of 300-600 tokens, decode rows over 128-1800 keys)."""
    gen = torch.Generator().manual_seed(94 + n_seq)
    pre = uniform_lens(gen, 6, 300, 600)
    dec = uniform_lens(gen, n_seq - 6, 128, 1800)
    nq, nk = pre + [1] * len(dec), pre + dec
    pool = sum((n + BLOCK - 1) // BLOCK for n in nk) + 3
    kc, vc, tables = paged_pool(gen, nk, pool)
    q = randn(gen, sum(nq), H, D)
    out = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq),
                                 max(nk), softmax_scale=SCALE, causal=True, block_table=tables.to(DEV))
    want = ref.varlen(q.float(), _cu(nq), _cu(nk), k_cache=kc, v_cache=vc, block_tables=tables)
    attn_close(out, want, f"{n_seq} sequences")


def test_mixed_launch_plan_recorded_then_reused_equals_unplanned():
    """The decode rows of a mixed launch plan like a decode step's layers: a call that records the layout and two
    that reuse it (the 28 layers of a mixed step share their lengths and tables) equal the unplanned call bit for
    bit."""
    from voxcpm2_arabic_dialects_turbo_amd.ops import forget_plans, varlen_attention

    gen = torch.Generator().manual_seed(95)
    nq, nk, kc, vc, tables = _mixed_case(gen, 120, 1800, uniform_lens(gen, 6, 300, 600), HK, block_size=BLOCK)
    q = randn(gen, sum(nq), H, D).to(DEV)
    kw = dict(cu_seqlens_q=_cu(nq).to(DEV), cu_seqlens_k=_cu(nk).to(DEV), max_seqlen_q=max(nq), softmax_scale=SCALE,
              causal=True, block_table=tables.to(DEV), k_cache=kc.to(DEV), v_cache=vc.to(DEV))
    forget_plans()
    plain = varlen_attention(q, None, None, **kw)
    planned = [varlen_attention(q, None, None, plan=("mixed plan test", 1), **kw) for _ in range(3)]
    torch.cuda.synchronize()
    forget_plans()
    for i, o in enumerate(planned):
        assert torch.equal(o, plain), f"call {i} ({'record' if i == 0 else 'reuse'}) differs from the unplanned one"
    want = ref.varlen(q.float().cpu(), _cu(nq), _cu(nk), k_cache=kc, v_cache=vc, block_tables=tables)
    attn_close(plain, want, "mixed launch, planned")


@pytest.mark.parametrize("case", ["config2", "short", "padded_slots", "one_kv_head", "unaligned_caches"])
def test_packed_prefill_with_the_store_riding_in_it_equals_store_then_prefill(case):
    """prefill_attention_store (the store copied by the attention launch's last workgroups) against store_kvcache
    then the packed varlen prefill on the same inputs: outputs and both caches bit-identical, the outputs within
    tolerance of the oracle. Cases: config 2 (8 x U[64, 512]); many short sequences (a grid of fewer than 256
    workgroups, each copying several rows); padding slots (-1) and slots past the cache, which store nothing;
    one kv head; caches that are not 16-byte aligned (the two-call form)."""
    from voxcpm2_arabic_dialects_turbo_amd.ops import prefill_attention_store

    gen = torch.Generator().manual_seed(96)
    hk = 1 if case == "one_kv_head" else HK
    lens = uniform_lens(gen, 40, 1, 30) if case == "short" else uniform_lens(gen, 8, 64, 512)
    T = sum(lens)
    kc, vc, tables = paged_pool(gen, lens, 512, hk=hk)
    qkv = randn(gen, T, (H + 2 * hk) * D).to(DEV)
    q, k, v = qkv.split([H * D, hk * D, hk * D], dim=-1)
    q, k, v = q.view(T, H, D), k.view(T, hk, D), v.view(T, hk, D)
    slots = torch.cat([torch.tensor([ref.slot_of(tables[b].tolist(), j, BLOCK) for j in range(n)])
                       for b, n in enumerate(lens)]).to(torch.int32)
    if case == "padded_slots":
        slots[::7] = -1
        slots[3::11] = 512 * BLOCK + 5  # past the cache
    cu = _cu(lens).to(DEV)
    kc1, vc1 = kc.to(DEV), vc.to(DEV)
    kc2, vc2 = kc1.clone(), vc1.clone()
    if case == "unaligned_caches":  # the same caches 8 bytes into their buffers
        def shifted(c):
            buf = torch.empty(c.numel() + 4, dtype=c.dtype, device=DEV)
            view = buf[4:].view(c.shape)
            view.copy_(c)
            return view
        kc1, vc1 = shifted(kc1), shifted(vc1)
    fused = prefill_attention_store(q, k, v, kc1, vc1, slots.to(DEV), cu_seqlens_q=cu, cu_seqlens_k=cu,
                                    max_seqlen_q=max(lens), softmax_scale=SCALE)
    store_kvcache(k, v, kc2, vc2, slots.to(DEV))
    two = flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), softmax_scale=SCALE, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(fused, two), f"{case}: outputs differ from store + prefill"
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), f"{case}: caches differ from store_kvcache's"
    want = ref.varlen(q.float().cpu(), _cu(lens), _cu(lens), k=k.cpu(), v=v.cpu())
    attn_close(fused, want, f"{case}: against the oracle")


def _step_with_new_rows(gen, pre, prefix, dec, hk, block_size, misalign=0):
    """A paged step: prefills of pre[i] new tokens over prefix[i] cached ones, and one-query decode rows over dec[i]
    keys (the last one new); caches, tables, the step's q / k / v rows (strided as the model's qkv split; with
    `misalign`, k and v instead contiguous rows that many elements into a buffer of their own) and the slots the
    tables give the new tokens' positions."""
    nq = list(pre) + [1] * len(dec)
    nk = [a + b for a, b in zip(pre, prefix)] + list(dec)
    pool = sum((n + block_size - 1) // block_size for n in nk) + 3
    kc, vc, tables = paged_pool(gen, nk, pool, block_size=block_size, hk=hk)
    T = sum(nq)
    q, k, v = randn(gen, T, (H + 2 * hk) * D).to(DEV).split([H * D, hk * D, hk * D], dim=-1)
    q, k, v = q.view(T, H, D), k.view(T, hk, D), v.view(T, hk, D)
    if misalign:
        kv = torch.empty(2 * T * hk * D + misalign, dtype=torch.bfloat16, device=DEV)
        k2, v2 = kv[misalign:].view(2, T, hk, D)
        k2.copy_(k)
        v2.copy_(v)
        k, v = k2, v2
    slots = torch.tensor([ref.slot_of(tables[b].tolist(), j, block_size)
                          for b in range(len(nk)) for j in range(nk[b] - nq[b], nk[b])], dtype=torch.int32)
    return nq, nk, kc, vc, tables, q, k, v, slots


@pytest.mark.parametrize("case", ["config5", "prefixes", "one_kv_head", "unaligned_rows", "planned", "dense",
                                  "dense_8_waves", "dense_128_rows", "dense_blocks_of_512", "blocks_of_128",
                                  "blocks_of_32"])
def test_paged_prefill_with_the_store_riding_in_it_equals_store_then_prefill(case):
    """prefill_attention_store with a block table (the launch reads each sequence's new keys from the rows and
    writes the caches) against store_kvcache then flash_attn_varlen_func over the caches: outputs and both caches
    bit-identical, the outputs within tolerance of the oracle over the stored caches (calls of up to 4096 rows).
    Mixed launches (the merge kernel writes the caches): config 5 (6 prefills of U[300, 600] new tokens, 120 decode
    rows over U[128, 1800] keys, 256-token blocks); prefills over cached prefixes of 1-300 tokens, so that tiles
    straddle the first new key at every offset inside a 16-key piece and at piece edges (64-token blocks), beside
    decode rows; one kv head; the config 5 step over three layers with a plan (record, reuse, reuse). Key / value rows
    that are not 16-byte aligned take the two calls. Dense prefills (no decode rows; the prefill launch's last
    workgroups write the caches), with cached prefixes: the rank-major 64-row form, the 8-wave form and the 128-row
    form; 512-token blocks (dense) and 128-token blocks (with decode rows). 32-token blocks take the two calls."""
    from voxcpm2_arabic_dialects_turbo_amd.ops import prefill_attention_store

    gen = torch.Generator().manual_seed(97)
    hk = 1 if case == "one_kv_head" else HK
    if case in ("config5", "planned", "unaligned_rows", "one_kv_head"):
        pre, prefix, dec, bs = uniform_lens(gen, 6, 300, 600), [0] * 6, uniform_lens(gen, 120, 128, 1800), BLOCK
    elif case == "prefixes":
        prefix = [1, 15, 16, 17, 31, 48, 63, 64, 65, 100, 130, 255, 256, 300]
        pre, dec, bs = uniform_lens(gen, len(prefix), 2, 150), uniform_lens(gen, 60, 1, 700), 64
    elif case == "dense":  # 12 prefills of 100-200 tokens over prefixes, 4 decode rows (on the prefill kernel)
        prefix = [0, 1, 17, 64, 100, 255, 300, 5, 33, 128, 0, 70]
        pre, dec, bs = uniform_lens(gen, 12, 100, 200), uniform_lens(gen, 4, 10, 300), 64
    elif case == "dense_8_waves":  # 3 x ~2500 tokens: 128-row items, fewer than 2048 workgroups
        pre, prefix, dec, bs = uniform_lens(gen, 3, 2400, 2600), [0, 45, 300], [], BLOCK
    elif case == "dense_128_rows":  # 6 x ~5600 tokens: 128-row items, more than 2048 workgroups
        pre, prefix, dec, bs = uniform_lens(gen, 6, 5500, 5700), [0, 1, 64, 250, 256, 700], [], 64
    elif case == "dense_blocks_of_512":  # prefixes inside, at and past a block's first tile and its end
        pre, prefix, dec, bs = uniform_lens(gen, 6, 50, 300), [0, 7, 100, 511, 512, 700], [], 512
    elif case == "blocks_of_128":
        pre, prefix, bs = uniform_lens(gen, 6, 20, 250), [0, 13, 127, 128, 200, 333], 128
        dec = uniform_lens(gen, 40, 1, 900)
    else:  # blocks_of_32
        pre, prefix, dec, bs = uniform_lens(gen, 5, 50, 300), [0, 7, 40, 64, 90], uniform_lens(gen, 20, 1, 300), 32
    nq, nk, kc, vc, tables, q, k, v, slots = _step_with_new_rows(gen, pre, prefix, dec, hk, bs,
                                                                 misalign=4 if case == "unaligned_rows" else 0)
    cu_q, cu_k, bt, sl = _cu(nq).to(DEV), _cu(nk).to(DEV), tables.to(DEV), slots.to(DEV)
    kc1, vc1 = kc.to(DEV), vc.to(DEV)
    kc2, vc2 = kc1.clone(), vc1.clone()
    kw = dict(cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=max(nq), softmax_scale=SCALE, block_table=bt)
    fused = prefill_attention_store(q, k, v, kc1, vc1, sl, **kw)
    store_kvcache(k, v, kc2, vc2, sl)
    two = flash_attn_varlen_func(q, kc2, vc2, cu_q, cu_k, max(nq), max(nk), softmax_scale=SCALE, causal=True,
                                 block_table=bt)
    torch.cuda.synchronize()
    assert torch.equal(fused, two), f"{case}: outputs differ from store + prefill"
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), f"{case}: caches differ from store_kvcache's"
    if case == "planned":
        for i in range(3):
            o = prefill_attention_store(q, k, v, kc1, vc1, sl, plan=("riding store plan test", 1), **kw)
            torch.cuda.synchronize()
            assert torch.equal(o, fused), f"layer {i} ({'record' if i == 0 else 'reuse'}) differs"
        assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    if sum(nq) <= 4096:
        want = ref.varlen(q.float().cpu(), _cu(nq), _cu(nk), k_cache=kc2.cpu(), v_cache=vc2.cpu(),
                          block_tables=tables)
        attn_close(fused, want, f"{case}: against the oracle")


def test_mixed_step_with_the_riding_store_replays_in_a_hip_graph():
    """Attention.forward over a mixed step with caches (the store riding in the mixed launch) captured in a HIP graph
    and replayed three times, with eager calls on other queries between the replays: every replay equals the eager
    output bit for bit, and the caches hold the stored rows."""
    from voxcpm2_arabic_dialects_turbo_amd.context import reset_context, set_context
    from voxcpm2_arabic_dialects_turbo_amd.layers import Attention

    gen = torch.Generator().manual_seed(98)
    nq, nk, kc, vc, tables, q, k, v, slots = _step_with_new_rows(gen, [200, 333], [0, 70], [900, 5, 1500, 64], HK,
                                                                 BLOCK)
    layer = Attention(H, D, SCALE, HK)
    layer.k_cache, layer.v_cache = kc.to(DEV), vc.to(DEV)
    kc_want, vc_want = layer.k_cache.clone(), layer.v_cache.clone()
    store_kvcache(k, v, kc_want, vc_want, slots.to(DEV))
    q2 = randn(gen, *q.shape).to(DEV)
    try:
        set_context(True, _cu(nq).to(DEV), _cu(nk).to(DEV), max(nq), max(nk), slots.to(DEV), None, tables.to(DEV))
        eager = layer(q, k, v)
        eager2 = layer(q2, k, v)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            static = layer(q, k, v)
        for r in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(static, eager), f"replay {r}"
            other = layer(q2, k, v)
            torch.cuda.synchronize()
            assert torch.equal(other, eager2)
        assert torch.equal(layer.k_cache, kc_want) and torch.equal(layer.v_cache, vc_want)
    finally:
        reset_context()
