"""GPU parity of the split-KV paged decode kernel (HIP kernel 3) against the oracle (fp32 on the same bf16 inputs):
max-abs <= 2e-2 and mean-abs <= 2e-3."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import attention as ref
from tests._util import BLOCK, D, H, HK, attn_close, paged_pool, randn, uniform_lens
from tests.golden import make_golden
from voxcpm2_arabic_dialects_turbo_amd import _lib
from voxcpm2_arabic_dialects_turbo_amd.ops import decode_attention, flash_attn_with_kvcache

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = D ** -0.5


def _check(q, kc, vc, lens, tables, what, h=H, hk=HK):
    out = decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV),
                           tables.to(DEV), SCALE)
    torch.cuda.synchronize()
    want = ref.decode(q.float().cpu(), kc, vc, lens, tables, SCALE)
    return attn_close(out, want, what), out


def test_decode_config1_golden():
    """benchmark config 1 (1 sequence, context 512, 4 shuffled blocks), inputs rounded to bf16 on the GPU."""
    inp = make_golden.inputs("decode_c1")
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"), allow_pickle=False)
    q, kc, vc = inp["q"].bfloat16(), inp["k_cache"].bfloat16(), inp["v_cache"].bfloat16()
    _, out = _check(q, kc, vc, inp["lens"].tolist(), inp["tables"], "config 1")
    attn_close(out, torch.from_numpy(g["decode_c1__out"]), "config 1 vs golden (fp32 inputs)")


def test_decode_config3_shape():
    """benchmark config 3: 40 sequences, contexts U[200, 1500], 1024-block pool."""
    gen = torch.Generator().manual_seed(30)
    lens = uniform_lens(gen, 40, 200, 1500)
    kc, vc, tables = paged_pool(gen, lens, 1024)
    _check(randn(gen, 40, H, D), kc, vc, lens, tables, "config 3")


def test_decode_ragged_contexts_and_stale_table_columns():
    """Context lengths around every tile / chunk / block boundary; columns past a row's blocks hold garbage ids
    (as captured graph buffers do) and must never be read."""
    gen = torch.Generator().manual_seed(31)
    lens = [1, 2, 31, 32, 33, 127, 128, 129, 255, 256, 257, 383, 511, 512, 513, 1000, 2047, 2048]
    kc, vc, tables = paged_pool(gen, lens, 160, extra_cols=2)
    tables[tables < 0] = 10 ** 9  # stale ids far outside the pool
    tables[0, -1] = -7
    _check(randn(gen, len(lens), H, D), kc, vc, lens, tables, "ragged")


def test_decode_padded_rows_write_zeros():
    gen = torch.Generator().manual_seed(32)
    lens = [300, 0, 5, 0]
    kc, vc, tables = paged_pool(gen, [300, 1, 5, 1], 8)
    (_, _), out = _check(randn(gen, 4, H, D), kc, vc, lens, tables, "padded")
    assert int(out[1].abs().sum()) == 0 and int(out[3].abs().sum()) == 0


def test_decode_one_kv_head_tp2_shape():
    """Tensor parallel 2 splits heads: 8 query heads over 1 KV head."""
    gen = torch.Generator().manual_seed(33)
    lens = uniform_lens(gen, 12, 1, 1200)
    kc, vc, tables = paged_pool(gen, lens, 64, hk=1)
    _check(randn(gen, 12, 8, D), kc, vc, lens, tables, "HK=1")


@pytest.mark.parametrize("h,hk", [(1, 1), (2, 2), (4, 2), (6, 2), (10, 2), (13, 1), (16, 1)])
def test_decode_every_group_size(h, hk):
    """Any num_heads <= 16 over 1 or 2 kv heads (the ABI's contract): groups 1, 2, 3, 5, 13 and 16 besides the
    model's 8. Heads past num_heads pad the 16 query columns of the MFMA tiles and must neither leak into the real
    heads nor be written; contexts from 0 to beyond one workgroup's range (sequences cut by range boundaries)."""
    gen = torch.Generator().manual_seed(70 + 3 * h + hk)
    lens = [0, 1, 17, 256, 700] + uniform_lens(gen, 20, 1, 3000)
    kc, vc, tables = paged_pool(gen, [max(n, 1) for n in lens], 400, hk=hk)
    (_, _), out = _check(randn(gen, len(lens), h, D), kc, vc, lens, tables, f"{h}/{hk} heads", h=h, hk=hk)
    assert out.shape == (len(lens), h, D) and int(out[0].abs().sum()) == 0


@pytest.mark.parametrize("bs", [96, 128, 512, 1024])
def test_decode_block_sizes(bs):
    """Block sizes the ABI accepts beside 32, 64 and 256 (any multiple of 32; 96 is not a power of two, so 16-token
    steps start at every offset of a block): contexts around block boundaries and beyond one workgroup's range."""
    gen = torch.Generator().manual_seed(80 + bs)
    lens = [1, bs - 1, bs, bs + 1, 2 * bs + 17] + uniform_lens(gen, 16, 1, 4000)
    kc, vc, tables = paged_pool(gen, lens, sum(-(-n // bs) for n in lens) + 3, block_size=bs)
    _check(randn(gen, len(lens), H, D), kc, vc, lens, tables, f"block size {bs}")


def test_decode_strided_query_rows_and_small_blocks():
    """q as a view of the qkv output (rows 2560 elements apart); 64-token blocks."""
    gen = torch.Generator().manual_seed(34)
    lens = uniform_lens(gen, 9, 1, 900)
    kc, vc, tables = paged_pool(gen, lens, 200, block_size=64)
    qkv = randn(gen, 9, (H + 2 * HK) * D)
    q = qkv.to(DEV)[:, :H * D].view(9, H, D)
    assert q.stride(0) == (H + 2 * HK) * D
    out = decode_attention(q, kc.to(DEV), vc.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV),
                           tables.to(DEV), SCALE)
    attn_close(out, ref.decode(q.float().cpu(), kc, vc, lens, tables, SCALE), "strided q")


@pytest.mark.parametrize("grid", [1, 2, 7, 64, 333, 768, 4000])
def test_decode_split_grids_agree(grid):
    """The split kernel's range partition at many grid sizes: one workgroup holding every sequence, ranges cutting
    sequences anywhere, more workgroups than steps (the launch then uses one per step)."""
    gen = torch.Generator().manual_seed(35)
    lens = uniform_lens(gen, 20, 1, 2048) + [0, 64, 65]
    kc, vc, tables = paged_pool(gen, [max(n, 1) for n in lens], 200)
    lib = _lib.load()
    lib.vox_set_decode_workgroups(grid)
    try:
        (_, _), out = _check(randn(gen, len(lens), H, D), kc, vc, lens, tables, f"grid {grid}")
        assert int(out[20].abs().sum()) == 0
    finally:
        lib.vox_set_decode_workgroups(0)


@pytest.mark.parametrize("grid", [1, 3, 256])
def test_decode_sparse_batch_of_mostly_empty_rows(grid):
    """300 rows, most of them empty (padded): the split kernel's rounds look sequences up in windows of 64 rows, so
    a round can end at a window's last non-empty row before the workgroup's range does (runs of 60+ empty rows),
    and elsewhere at eight non-empty rows (the dense run 200-210)."""
    gen = torch.Generator().manual_seed(41)
    lens = [0] * 300
    for i in (5, 70, 71, 72, 140, 141, 299) + tuple(range(200, 211)):
        lens[i] = int(torch.randint(1, 1500, (1,), generator=gen))
    kc, vc, tables = paged_pool(gen, [max(n, 1) for n in lens], 400)
    lib = _lib.load()
    lib.vox_set_decode_workgroups(grid)
    try:
        (_, _), out = _check(randn(gen, len(lens), H, D), kc, vc, lens, tables, f"sparse, grid {grid}")
    finally:
        lib.vox_set_decode_workgroups(0)
    empty = torch.tensor([n == 0 for n in lens], device=out.device)
    assert int(out[empty].abs().sum()) == 0


@pytest.mark.parametrize("lens", [[16384], [4096] * 4, [300] * 16 + [8192], [5, 9000, 3, 0, 2100, 64]],
                         ids=["1x16384", "4x4096", "16x300+8192", "mixed"])
def test_decode_few_long_sequences(lens):
    """Few sequences, some far longer than a workgroup's share of the steps: the launch then uses fewer workgroups
    (no sequence is cut into more than about 32 partials) and the merge kernel folds the partials of one sequence in
    several batches of loads."""
    gen = torch.Generator().manual_seed(40)
    pool = sum((max(n, 1) + BLOCK - 1) // BLOCK for n in lens) + 4
    kc, vc, tables = paged_pool(gen, [max(n, 1) for n in lens], pool)
    (_, _), out = _check(randn(gen, len(lens), H, D), kc, vc, lens, tables, f"lens {lens[:6]}")
    for i, n in enumerate(lens):
        if n == 0:
            assert int(out[i].abs().sum()) == 0


def test_decode_repeated_calls_of_changing_batch():
    """Back-to-back calls that reuse the workspace with different batch sizes and split counts."""
    gen = torch.Generator().manual_seed(36)
    for n in (30, 7, 30, 64):
        lens = uniform_lens(gen, n, 100, 2048)
        kc, vc, tables = paged_pool(gen, lens, 8 * n)
        _check(randn(gen, n, H, D), kc, vc, lens, tables, f"batch {n}")


def test_decode_block_table_wider_than_lds():
    """A block table of more entries than the kernel keeps in LDS (here 40 x 128 columns) is read from memory."""
    gen = torch.Generator().manual_seed(39)
    lens = uniform_lens(gen, 40, 1, 128 * 32)
    kc, vc, tables = paged_pool(gen, lens, 40 * 128, block_size=32, extra_cols=128)
    tables = tables[:, :128].contiguous()
    tables[tables < 0] = 7
    _check(randn(gen, 40, H, D), kc, vc, lens, tables, "wide table")


def test_decode_batch_beyond_one_launch():
    """More sequences than one launch's step layout holds (512): the call runs consecutive launches."""
    gen = torch.Generator().manual_seed(38)
    lens = uniform_lens(gen, 1100, 0, 300)
    kc, vc, tables = paged_pool(gen, [max(n, 1) for n in lens], 1300, block_size=256)
    _check(randn(gen, len(lens), H, D), kc, vc, lens, tables, "batch 1100")


def test_decode_config4_layer_full_size():
    """benchmark config 4, one layer at full size: 150 sequences, contexts U[256, 2048], 2048-block pool."""
    gen = torch.Generator().manual_seed(100)
    lens = uniform_lens(gen, 150, 256, 2048)
    kc, vc, tables = paged_pool(gen, lens, 2048)
    _check(randn(gen, 150, H, D), kc, vc, lens, tables, "config 4 layer")


def test_with_kvcache_entry_point_shapes():
    """flash_attn_with_kvcache: [B, 1, H, D] decode and a [B, 3, H, D] multi-token query (bottom-right causal)."""
    gen = torch.Generator().manual_seed(37)
    lens = [40, 300, 257]
    kc, vc, tables = paged_pool(gen, lens, 8)
    q = randn(gen, 3, 1, H, D)
    args = dict(cache_seqlens=torch.tensor(lens, dtype=torch.int32, device=DEV), block_table=tables.to(DEV),
                softmax_scale=SCALE, causal=True)
    out = flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.to(DEV), **args)
    assert out.shape == (3, 1, H, D)
    attn_close(out[:, 0], ref.decode(q[:, 0].float(), kc, vc, lens, tables, SCALE), "with_kvcache Lq=1")
    q3 = randn(gen, 3, 3, H, D)
    out3 = flash_attn_with_kvcache(q3.to(DEV), kc.to(DEV), vc.to(DEV), **args)
    want = ref.varlen(q3.reshape(9, H, D).float(), [0, 3, 6, 9], [0, 40, 340, 597], k_cache=kc, v_cache=vc,
                      block_tables=tables)
    attn_close(out3.reshape(9, H, D), want, "with_kvcache Lq=3")


def test_decode_closed_forms_identical_keys_and_one_token():
    """Closed forms that pin the kernel without the oracle: with every key of a sequence identical the softmax is
    uniform and o = mean(V) over the context; with a one-token context o = V[0] exactly (p = 1)."""
    gen = torch.Generator().manual_seed(39)
    lens = [1, 300, 513, 64]
    kc, vc, tables = paged_pool(gen, lens, 40)
    key = randn(gen, HK, D)
    for b, n in enumerate(lens):  # the same key in every slot a sequence uses
        for j in range(n):
            blk, off = tables[b, j // BLOCK].item(), j % BLOCK
            kc[blk, off] = key
    q = randn(gen, len(lens), H, D)
    out = decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV),
                           tables.to(DEV), SCALE).float().cpu()
    for b, n in enumerate(lens):
        rows = torch.stack([vc[tables[b, j // BLOCK], j % BLOCK] for j in range(n)]).float()  # [n, HK, D]
        want = rows.mean(0).repeat_interleave(H // HK, dim=0)  # head h reads kv head h // 8
        err = (out[b] - want).abs().max().item()
        assert err <= (0.0 if n == 1 else 2e-2), f"sequence {b} (ctx {n}): max-abs {err}"


def test_decode_equals_varlen_prefill_with_one_query():
    """A decode step and a paged varlen call with one query per sequence (nq = 1, nk = ctx) compute the same
    attention on different kernels; they agree within the attention tolerance."""
    from voxcpm2_arabic_dialects_turbo_amd.ops import flash_attn_varlen_func

    gen = torch.Generator().manual_seed(40)
    lens = uniform_lens(gen, 24, 1, 1800)
    kc, vc, tables = paged_pool(gen, lens, 200)
    q = randn(gen, len(lens), H, D).to(DEV)
    kc_d, vc_d, t_d = kc.to(DEV), vc.to(DEV), tables.to(DEV)
    dec = decode_attention(q, kc_d, vc_d, torch.tensor(lens, dtype=torch.int32, device=DEV), t_d, SCALE)
    cu_q = torch.arange(len(lens) + 1, dtype=torch.int32, device=DEV)
    cu_k = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32, device=DEV)
    pre = flash_attn_varlen_func(q, kc_d, vc_d, cu_q, cu_k, 1, max(lens), softmax_scale=SCALE, causal=True,
                                 block_table=t_d)
    attn_close(dec.float().cpu(), pre.float().cpu(), "decode vs varlen nq=1")


def test_unmapped_blocks_inside_the_context_are_masked_like_prefill():
    """A block-table entry inside a sequence's context that addresses no block (-1, or past the pool) takes no
    weight in decode (expected: the oracle over the sequence without that block's keys; a fully unmapped context
    gives zeros), and the one-query varlen prefill over the same bad table gives the same result."""
    from voxcpm2_arabic_dialects_turbo_amd.ops import flash_attn_varlen_func

    gen = torch.Generator().manual_seed(39)
    lens = [700, 300, 200, 1000]
    pool = 16
    kc, vc, tables = paged_pool(gen, lens, pool)
    bad = tables.clone()
    bad[0, 1] = -1          # keys 256 .. 511 of sequence 0
    bad[1, 0] = pool + 3    # keys 0 .. 255 of sequence 1
    bad[2, 0] = -9          # all of sequence 2
    q = randn(gen, len(lens), H, D)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=DEV)
    out = decode_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), lens_d, bad.to(DEV), SCALE)
    width = tables.shape[1]
    keep = [[int(x) for j, x in enumerate(tables[b].tolist()) if x >= 0 and bad[b, j] == x] for b in range(4)]
    t_ref = torch.tensor([k + [-1] * (width - len(k)) for k in keep], dtype=torch.int32)
    lens_ref = [lens[0] - 256, lens[1] - 256, 0, lens[3]]
    want = ref.decode(q.float(), kc, vc, lens_ref, t_ref, SCALE)
    attn_close(out, want, "decode, unmapped blocks masked")
    assert out[2].float().abs().max().item() == 0.0
    cu_q = torch.arange(len(lens) + 1, dtype=torch.int32, device=DEV)
    cu_k = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32, device=DEV)
    pre = flash_attn_varlen_func(q.to(DEV), kc.to(DEV), vc.to(DEV), cu_q, cu_k, 1, max(lens), softmax_scale=SCALE,
                                 causal=True, block_table=bad.to(DEV))
    attn_close(pre, out.float(), "prefill nq=1 vs decode on the same unmapped blocks")


def _store_then_decode(q, key, value, slots, kc, vc, lens, tables):
    """The two-call reference of the store mode: store_kvcache, then decode, on copies of the caches."""
    from voxcpm2_arabic_dialects_turbo_amd.ops import store_kvcache

    k2, v2 = kc.clone(), vc.clone()
    store_kvcache(key, value, k2, v2, slots)
    return decode_attention(q, k2, v2, lens, tables, SCALE), k2, v2


@pytest.mark.parametrize("case", ["last_token", "middle_slot", "one_kv_head", "wide_table", "two_launches"])
def test_decode_with_the_store_matches_store_then_decode(case):
    """The decode call with the step's store folded in (vox_decode_attn_store) against store_kvcache followed by
    decode_attention: outputs and caches bit-identical. The new token at each sequence's last position (the
    engine's layout), or at a slot in the middle of its own context; padded rows (context 0, slot -1); one KV head;
    a block table too wide for LDS; more sequences than one launch takes. Key / value rows are strided views of a
    fused qkv row, as the model hands them over."""
    gen = torch.Generator().manual_seed(91)
    hk = 1 if case == "one_kv_head" else HK
    h = 8 if case == "one_kv_head" else H
    B = {"wide_table": 512, "two_launches": 600}.get(case, 150)
    lens = uniform_lens(gen, B, 1, {"two_launches": 700, "wide_table": 600}.get(case, 2048))
    lens[3] = 0  # a padded row
    bs = 256 if case != "wide_table" else 32
    kc, vc, tables = paged_pool(gen, lens, sum(-(-max(n, 1) // bs) for n in lens) + 4, block_size=bs, hk=hk)
    qkv = randn(gen, B, (h + 2 * hk) * D).to(DEV)
    q, key, value = qkv.split([h * D, hk * D, hk * D], dim=-1)
    q, key, value = q.view(B, h, D), key.view(B, hk, D), value.view(B, hk, D)
    slots = []
    for b, n in enumerate(lens):
        if n == 0:
            slots.append(-1)
            continue
        pos = n - 1 if case != "middle_slot" else (n - 1) // 2
        slots.append(int(tables[b, pos // bs]) * bs + pos % bs)
    slots = torch.tensor(slots, dtype=torch.int32, device=DEV)
    kc, vc, tables = kc.to(DEV), vc.to(DEV), tables.to(DEV)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=DEV)
    want, k_want, v_want = _store_then_decode(q, key, value, slots, kc, vc, lens_d, tables)
    k1, v1 = kc.clone(), vc.clone()
    got = decode_attention(q, k1, v1, lens_d, tables, SCALE, key=key, value=value, slot_mapping=slots)
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"{case}: outputs differ from store + decode"
    assert torch.equal(k1, k_want) and torch.equal(v1, v_want), f"{case}: caches differ from store_kvcache's"


def test_decode_with_the_store_in_a_hip_graph_replays_like_eager():
    """Store mode captured in a HIP graph and replayed over changing inputs (new tokens, positions and slots
    written into the captured buffers), each replay against the two-call form run eagerly."""
    gen = torch.Generator().manual_seed(92)
    B, pool = 64, 600
    lens = uniform_lens(gen, B, 100, 1500)
    kc, vc, tables_h = paged_pool(gen, [n + 8 for n in lens], pool)
    kc, vc, tables = kc.to(DEV), vc.to(DEV), tables_h.to(DEV)
    q = torch.zeros(B, H, D, dtype=torch.bfloat16, device=DEV)
    key = torch.zeros(B, HK, D, dtype=torch.bfloat16, device=DEV)
    value = torch.zeros_like(key)
    lens_d = torch.zeros(B, dtype=torch.int32, device=DEV)
    slots = torch.zeros(B, dtype=torch.int32, device=DEV)
    out = torch.empty(B, H, D, dtype=torch.bfloat16, device=DEV)
    k1, v1 = kc.clone(), vc.clone()

    def load(step):
        n = torch.tensor([x + step for x in lens], dtype=torch.int32)
        s = torch.tensor([int(tables_h[b, (int(n[b]) - 1) // BLOCK]) * BLOCK + (int(n[b]) - 1) % BLOCK
                          for b in range(B)], dtype=torch.int32)
        q.copy_(randn(gen, B, H, D))
        key.copy_(randn(gen, B, HK, D))
        value.copy_(randn(gen, B, HK, D))
        lens_d.copy_(n)
        slots.copy_(s)

    load(0)
    decode_attention(q, k1, v1, lens_d, tables, SCALE, out=out, key=key, value=value, slot_mapping=slots)
    k_ref, v_ref = k1.clone(), v1.clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        decode_attention(q, k1, v1, lens_d, tables, SCALE, out=out, key=key, value=value, slot_mapping=slots)
    for step in range(1, 5):
        load(step)
        want, k_ref, v_ref = _store_then_decode(q, key, value, slots, k_ref, v_ref, lens_d, tables)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {step}: output"
        assert torch.equal(k1, k_ref) and torch.equal(v1, v_ref), f"replay {step}: caches"


def _layers_of_one_step(gen, lens, n_layers, bs=BLOCK, store=False, width_extra=0):
    """n_layers layers of one decode step: shared lengths, tables (and slots), per-layer caches, q (and new rows)."""
    pool = sum(-(-max(n, 1) // bs) for n in lens) + 4
    _, _, tables = paged_pool(gen, lens, pool, block_size=bs, extra_cols=width_extra)
    layers = []
    for _ in range(n_layers):
        kc, vc = randn(gen, pool, bs, HK, D), randn(gen, pool, bs, HK, D)
        qkv = randn(gen, len(lens), (H + 2 * HK) * D).to(DEV)
        layers.append((kc.to(DEV), vc.to(DEV), qkv))
    slots = [int(tables[b, (n - 1) // bs]) * bs + (n - 1) % bs if n > 0 else -1 for b, n in enumerate(lens)]
    return layers, tables.to(DEV), torch.tensor(lens, dtype=torch.int32, device=DEV), \
        torch.tensor(slots, dtype=torch.int32, device=DEV)


def _run_step(layers, tables, lens, slots, plan, store):
    outs, caches = [], []
    for kc, vc, qkv in layers:
        B = qkv.shape[0]
        q, k, v = qkv.split([H * D, HK * D, HK * D], dim=-1)
        k1, v1 = kc.clone(), vc.clone()
        kw = dict(key=k.view(B, HK, D), value=v.view(B, HK, D), slot_mapping=slots) if store else {}
        outs.append(decode_attention(q.view(B, H, D), k1, v1, lens, tables, SCALE, plan=plan, **kw))
        caches.append((k1, v1))
    torch.cuda.synchronize()
    return outs, caches


@pytest.mark.parametrize("store", [False, True])
def test_plan_recorded_by_the_first_layer_and_reused_by_the_others(store):
    """A decode step whose plan (the layout: each workgroup's range, sequences and tile block ids) is recorded by
    the first layer's call and reused by the next ones gives the unplanned calls' outputs bit for bit (and, with the
    store folded in, the same caches), and every layer matches the oracle."""
    from voxcpm2_arabic_dialects_turbo_amd import ops

    gen = torch.Generator().manual_seed(150)
    lens = uniform_lens(gen, 150, 256, 2048)
    lens[7] = 0
    layers, tables, lens_d, slots = _layers_of_one_step(gen, lens, 4, store=store)
    ops.forget_plans()
    planned, pc = _run_step(layers, tables, lens_d, slots, ("step", 1), store)
    plain, cc = _run_step(layers, tables, lens_d, slots, None, store)
    for i in range(len(layers)):
        assert torch.equal(planned[i], plain[i]), f"layer {i}: planned call differs from the unplanned one"
        assert torch.equal(pc[i][0], cc[i][0]) and torch.equal(pc[i][1], cc[i][1])
    kc, vc, qkv = layers[2]
    q, k, v = qkv.split([H * D, HK * D, HK * D], dim=-1)
    kc2, vc2 = kc.cpu(), vc.cpu()
    if store:
        ref.store_kvcache(k.view(-1, HK, D).cpu(), v.view(-1, HK, D).cpu(), kc2, vc2, slots.cpu())
    attn_close(planned[2], ref.decode(q.view(-1, H, D).float().cpu(), kc2, vc2, lens, tables.cpu(), SCALE),
               "planned layer 2")


@pytest.mark.parametrize("grid, lens", [(2, [700] * 60), (1, [40] * 100 + [3000]), (5, [1] * 300 + [2048] * 3)],
                         ids=["range_beyond_a_record", "window_beyond_64_sequences", "many_rounds"])
def test_plan_records_that_cannot_hold_a_range_fall_back_to_the_scan(grid, lens):
    """Ranges longer than a record holds, or touching more than the 64 sequences of its window, are recorded as
    unusable; reusing the plan then scans the layout again in those workgroups: same bits as unplanned calls."""
    from voxcpm2_arabic_dialects_turbo_amd import ops

    lib = _lib.load()
    lib.vox_set_decode_workgroups(grid)
    try:
        gen = torch.Generator().manual_seed(151)
        layers, tables, lens_d, slots = _layers_of_one_step(gen, lens, 3)
        ops.forget_plans()
        planned, _ = _run_step(layers, tables, lens_d, slots, ("fallback", grid), False)
        plain, _ = _run_step(layers, tables, lens_d, slots, None, False)
    finally:
        lib.vox_set_decode_workgroups(0)
    for i in range(len(layers)):
        assert torch.equal(planned[i], plain[i]), f"layer {i}"
    kc, vc, qkv = layers[1]
    attn_close(planned[1], ref.decode(qkv[:, :H * D].view(-1, H, D).float().cpu(), kc.cpu(), vc.cpu(), lens,
                                      tables.cpu(), SCALE), "fallback layer 1")
