"""Host logic on the CPU: the context builders against the oracle's per-token loops, the staging buffer, KV-cache
allocation, decode graph buffers, and Attention.forward's dispatch (with the kernels recorded, not run)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import context as ctxref
from voxcpm2_arabic_dialects_turbo_amd import layers, runner
from voxcpm2_arabic_dialects_turbo_amd.context import get_context, reset_context, set_context
from voxcpm2_arabic_dialects_turbo_amd.layers import Attention

BS = 4  # small blocks: prefixes end inside blocks, sequences span several (as the reference's host tests do)


@pytest.fixture(autouse=True)
def _clean_context():
    reset_context()
    yield
    reset_context()


def _tasks(rng, n, warmup=False, block_size=BS):
    tasks, next_block = [], 0
    for i in range(n):
        length = int(rng.integers(1, 15))
        cached = 0 if warmup else int(rng.integers(0, length))
        blocks = [] if warmup else list(range(next_block, next_block + (length + block_size - 1) // block_size))
        next_block += len(blocks) + int(rng.integers(0, 3))
        tasks.append(runner.RunnerTask(blocks, length, cached, block_size, seq_id=f"s{i}"))
    return tasks


def _snapshot():
    c = get_context()
    out = {"max": (c.is_prefill, c.max_seqlen_q, c.max_seqlen_k)}
    for f in ("cu_seqlens_q", "cu_seqlens_k", "slot_mapping", "block_tables", "context_lens"):
        v = getattr(c, f)
        out[f] = None if v is None else (v.dtype, v.tolist())
    return out


@pytest.mark.parametrize("seed,warmup,graphs", [(0, False, False), (1, False, True), (2, True, False), (3, False, False),
                                                (4, True, True)])
def test_prefill_context_matches_the_per_token_loop(seed, warmup, graphs):
    rng = np.random.default_rng(seed)
    tasks = _tasks(rng, 9, warmup=warmup)
    positions = runner.prepare_prefill_context(tasks, BS, device="cpu", graphs=graphs)
    got = _snapshot()
    pos, cu_q, cu_k, max_q, max_k, slots, tables = ctxref.prefill_context(BS, tasks, graphs=graphs)
    assert (positions.dtype, positions.tolist()) == (torch.int64, pos)
    assert got["cu_seqlens_q"] == (torch.int32, cu_q) and got["cu_seqlens_k"] == (torch.int32, cu_k)
    assert got["max"] == (True, max_q, max_k)
    assert got["slot_mapping"] == (torch.int32, slots)
    assert got["block_tables"] == (None if tables is None else (torch.int32, tables))
    assert got["context_lens"] is None


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_decode_context_matches_the_per_sequence_formulas(seed):
    rng = np.random.default_rng(seed)
    tasks = _tasks(rng, 11)
    for t in tasks:  # decode: everything but the new token is cached
        t.num_cached_tokens = t.seq_length - 1
    positions = runner.prepare_decode_context(tasks, BS, device="cpu")
    got = _snapshot()
    pos, slots, lens, tables = ctxref.decode_context(BS, tasks)
    assert (positions.dtype, positions.tolist()) == (torch.int64, pos)
    assert got["slot_mapping"] == (torch.int32, slots)
    assert got["context_lens"] == (torch.int32, lens)
    assert got["block_tables"] == (torch.int32, tables)
    assert got["max"] == (False, 0, 0)


def test_step_staging_round_trips_dtypes_shapes_and_alignment():
    stage = runner.StepStaging("cpu")
    a = np.arange(5, dtype=np.int64)
    b = np.arange(7, dtype=np.int32)
    c = np.arange(12, dtype=np.int32).reshape(3, 4) - 6
    va, vb, vc, ve = stage.layout([(np.int64, a.shape), (np.int32, b.shape), (np.int32, c.shape), (np.int32, (0,))])
    va[:], vb[:], vc[...] = a, b, c
    ta, tb, tc, te = stage.upload()
    assert ta.dtype == torch.int64 and ta.tolist() == a.tolist()
    assert tb.dtype == torch.int32 and tb.tolist() == b.tolist()
    assert tc.shape == (3, 4) and tc.tolist() == c.tolist()
    assert te.shape == (0,)
    base = ta.data_ptr()  # arrays start at 256-byte offsets of the one buffer
    assert (tb.data_ptr() - base) % 256 == 0 and (tc.data_ptr() - base) % 256 == 0
    # the uploaded copy does not alias the staging buffer: refilling it leaves earlier uploads alone
    vb2, = stage.layout([(np.int32, (7,))])
    vb2[:] = -1
    assert tb.tolist() == b.tolist()


@pytest.mark.parametrize("first,count", [([3, 10, 0, 7], [2, 0, 3, 1]), ([5], [0]), ([], []), ([0, 0], [4, 4])])
def test_runs_are_concatenated_aranges(first, count):
    f, c = np.array(first, dtype=np.int64), np.array(count, dtype=np.int64)
    want = [x for fi, ci in zip(first, count) for x in range(fi, fi + ci)]
    assert runner._runs(f, c).tolist() == want


def test_prefill_slots_with_a_prefix_ending_inside_a_block_and_sequences_without_tables():
    """Pieces of a sequence's new tokens split at block boundaries; sequences without a table (warm-up) or without
    new tokens add no slots."""
    tasks = [runner.RunnerTask([9, 4, 7], 11, 3, BS), runner.RunnerTask([], 5, 0, BS),
             runner.RunnerTask([2, 8], 6, 6, BS), runner.RunnerTask([5], 2, 0, BS)]
    got = runner.prefill_slots(runner._Batch.of(tasks), BS).tolist()
    want = [t.block_table[p // BS] * BS + p % BS for t in tasks if t.block_table
            for p in range(t.num_cached_tokens, t.seq_length)]
    assert got == want == [39, 16, 17, 18, 19, 28, 29, 30, 20, 21]


def test_prefill_context_of_two_hundred_requests_matches_the_loop():
    """A burst the size of the reference's host-path benchmark (200 cloned requests over a shared prefix)."""
    rng = np.random.default_rng(7)
    tasks = []
    for i in range(200):
        prefix = [1000 + j for j in range(3)]
        length = int(rng.integers(13, 40))
        own = list(range(4 * i, 4 * i + (length + BS - 1) // BS - 3))
        tasks.append(runner.RunnerTask(prefix + own, length, 12, BS))
    positions = runner.prepare_prefill_context(tasks, BS, device="cpu")
    pos, cu_q, cu_k, max_q, max_k, slots, tables = ctxref.prefill_context(BS, tasks)
    got = _snapshot()
    assert positions.tolist() == pos and got["slot_mapping"] == (torch.int32, slots)
    assert got["block_tables"] == (torch.int32, tables) and got["max"] == (True, max_q, max_k)


def test_allocate_kv_cache_assigns_layer_views():
    model = torch.nn.ModuleList([Attention(16, 128, 128 ** -0.5, 2) for _ in range(3)]
                                + [Attention(16, 128, 128 ** -0.5, 2, is_causal=False)])
    kv = runner.allocate_kv_cache(model, num_blocks=5, block_size=256, device="cpu")
    assert kv.shape == (3, 2, 5, 256, 2, 128) and kv.dtype == torch.bfloat16
    for i, m in enumerate(runner.causal_attention_modules(model)):
        assert m.k_cache.data_ptr() == kv[i, 0].data_ptr() and m.v_cache.data_ptr() == kv[i, 1].data_ptr()
        assert m.k_cache.is_contiguous() and m.k_cache.stride(1) == 256
    assert model[3].k_cache.numel() == 0  # non-causal layers get no cache
    assert runner.kv_cache_block_bytes(runner.causal_attention_modules(model), 256) == 3 * 2 * 256 * 2 * 128 * 2
    with pytest.raises(ValueError):
        runner.allocate_kv_cache(model, num_blocks=5, block_size=128, device="cpu")


def test_decode_graph_buffers_load_like_run_model():
    bufs = runner.DecodeGraphBuffers(8, 4, device="cpu")
    bufs.block_tables.fill_(77)  # stale columns from an earlier step stay
    set_context(False, slot_mapping=torch.tensor([5, 9], dtype=torch.int32),
                context_lens=torch.tensor([6, 10], dtype=torch.int32),
                block_tables=torch.tensor([[1, 2], [3, 4]], dtype=torch.int32))
    bufs.load()
    assert bufs.slot_mapping.tolist() == [5, 9] + [-1] * 6
    assert bufs.context_lens.tolist() == [6, 10] + [0] * 6
    assert bufs.block_tables[:2].tolist() == [[1, 2, 77, 77], [3, 4, 77, 77]]
    bufs.bind(4)
    assert get_context().context_lens.shape == (4,) and not get_context().is_prefill
    assert runner.graph_batch_sizes(40) == [1, 2, 4, 8, 16, 32, 40]


# --- Attention.forward dispatch (kernels recorded) -------------------------------------------------------------------

class _Recorder:
    def __init__(self, monkeypatch):
        self.calls = []
        for name in ("store_kvcache", "flash_attn_varlen_func", "flash_attn_with_kvcache", "flash_attn_func",
                     "decode_attention", "prefill_attention_store"):
            monkeypatch.setattr(layers, name, self._make(name))

    def _make(self, name):
        def fn(*args, **kwargs):
            self.calls.append((name, args, kwargs))
            return torch.zeros(args[0].shape) if name == "decode_attention" else "o"
        return fn


def test_prefill_without_prefix_stores_and_attends_over_the_step_kv_in_one_call(monkeypatch):
    """store_kvcache then flash_attn_varlen_func over the step's own k / v (reference layers.py:332-348): the
    attention reads the packed rows, so the store rides in the same call."""
    rec = _Recorder(monkeypatch)
    attn = Attention(16, 128, 0.125, 2)
    attn.k_cache, attn.v_cache = torch.zeros(2, 256, 2, 128), torch.zeros(2, 256, 2, 128)
    q, k, v = torch.zeros(5, 16, 128), torch.zeros(5, 2, 128), torch.zeros(5, 2, 128)
    cu = torch.tensor([0, 5], dtype=torch.int32)
    slots = torch.arange(5, dtype=torch.int32)
    set_context(True, cu, cu, 5, 5, slots, None, None)
    assert attn(q, k, v) == "o"
    ((n0, a0, kw0),) = rec.calls
    assert n0 == "prefill_attention_store" and a0[0] is q and a0[1] is k and a0[2] is v
    assert a0[3] is attn.k_cache and a0[4] is attn.v_cache and a0[5] is slots
    assert kw0 == dict(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=5, softmax_scale=0.125, causal=True,
                       block_table=None, plan=None)


def test_prefill_with_block_tables_stores_and_attends_through_the_tables_in_one_call(monkeypatch):
    """store_kvcache then flash_attn_varlen_func over the caches through the block tables (reference
    layers.py:332-348 with a prefix cache or a mixed step): one prefill_attention_store call with the table and the
    step's plan key."""
    rec = _Recorder(monkeypatch)
    attn = Attention(16, 128, 0.125, 2)
    attn.k_cache, attn.v_cache = torch.zeros(2, 256, 2, 128), torch.zeros(2, 256, 2, 128)
    bt = torch.tensor([[1, 0]], dtype=torch.int32)
    slots = torch.tensor([298, 299], dtype=torch.int32)
    set_context(True, torch.tensor([0, 2], dtype=torch.int32), torch.tensor([0, 300], dtype=torch.int32), 2, 300,
                slots, None, bt)
    q, k, v = torch.zeros(2, 16, 128), torch.zeros(2, 2, 128), torch.zeros(2, 2, 128)
    assert attn(q, k, v) == "o"
    ((n0, a0, kw0),) = rec.calls
    assert n0 == "prefill_attention_store" and a0[0] is q and a0[1] is k and a0[2] is v and a0[5] is slots
    assert a0[3] is attn.k_cache and a0[4] is attn.v_cache and kw0["block_table"] is bt
    assert kw0["plan"] is not None and kw0["max_seqlen_q"] == 2


def test_prefill_rows_the_riding_store_cannot_take_store_then_attend(monkeypatch):
    """Key / value rows whose heads are not contiguous, or a slot_mapping that is not one slot per row, take
    store_kvcache then flash_attn_varlen_func over the caches."""
    rec = _Recorder(monkeypatch)
    attn = Attention(16, 128, 0.125, 2)
    attn.k_cache, attn.v_cache = torch.zeros(2, 256, 2, 128), torch.zeros(2, 256, 2, 128)
    bt = torch.tensor([[1, 0]], dtype=torch.int32)
    set_context(True, torch.tensor([0, 2], dtype=torch.int32), torch.tensor([0, 300], dtype=torch.int32), 2, 300,
                torch.tensor([298, 299, 300], dtype=torch.int32), None, bt)
    attn(torch.zeros(2, 16, 128), torch.zeros(2, 2, 128), torch.zeros(2, 2, 128))
    assert [c[0] for c in rec.calls] == ["store_kvcache", "flash_attn_varlen_func"]
    _, a1, kw1 = rec.calls[1]
    assert a1[1] is attn.k_cache and a1[2] is attn.v_cache and kw1["block_table"] is bt
    rec.calls.clear()
    set_context(True, torch.tensor([0, 2], dtype=torch.int32), torch.tensor([0, 300], dtype=torch.int32), 2, 300,
                torch.tensor([298, 299], dtype=torch.int32), None, bt)
    k = torch.zeros(2, 128, 2).transpose(1, 2)  # heads 1 element apart
    attn(torch.zeros(2, 16, 128), k, k)
    assert [c[0] for c in rec.calls] == ["store_kvcache", "flash_attn_varlen_func"]


def test_warmup_prefill_without_caches_skips_the_store(monkeypatch):
    rec = _Recorder(monkeypatch)
    attn = Attention(16, 128, 0.125, 2)
    cu = torch.tensor([0, 3], dtype=torch.int32)
    set_context(True, cu, cu, 3, 3, torch.zeros(0, dtype=torch.int32), None, None)
    attn(torch.zeros(3, 16, 128), torch.zeros(3, 2, 128), torch.zeros(3, 2, 128))
    assert [c[0] for c in rec.calls] == ["flash_attn_varlen_func"]


def test_decode_stores_and_attends_in_one_call_with_an_unsqueezed_output(monkeypatch):
    """A decode step with caches: the store rides in the decode call (key / value / slot_mapping of the step), the
    output comes back [B, 1, H, D] as flash_attn_with_kvcache's does."""
    rec = _Recorder(monkeypatch)
    attn = Attention(16, 128, 0.125, 2)
    attn.k_cache, attn.v_cache = torch.zeros(2, 256, 2, 128), torch.zeros(2, 256, 2, 128)
    lens, bt = torch.tensor([7, 9], dtype=torch.int32), torch.tensor([[0], [1]], dtype=torch.int32)
    slots = torch.tensor([6, 264], dtype=torch.int32)
    set_context(False, slot_mapping=slots, context_lens=lens, block_tables=bt)
    q, k, v = torch.zeros(2, 16, 128), torch.zeros(2, 2, 128), torch.zeros(2, 2, 128)
    o = attn(q, k, v)
    [(n0, a0, kw0)] = rec.calls
    assert n0 == "decode_attention" and a0[0] is q and a0[1] is attn.k_cache and a0[2] is attn.v_cache
    assert a0[3] is lens and a0[4] is bt and a0[5] == 0.125
    assert kw0["key"] is k and kw0["value"] is v and kw0["slot_mapping"] is slots
    assert o.shape == (2, 1, 16, 128)


@pytest.mark.parametrize("layout", ["unaligned_rows", "odd_row_stride", "slot_count"])
def test_decode_rows_the_fused_store_cannot_read_take_store_then_decode(monkeypatch, layout):
    """The fused store reads the new rows with 16-byte loads: rows that are not 16-byte aligned or whose stride is not
    a multiple of 8 elements, and a slot_mapping that is not one slot per row, take store_kvcache and then the
    decode kernel instead (the reference accepts them: nanovllm_voxcpm/model/layers.py:290-305)."""
    rec = _Recorder(monkeypatch)
    attn = Attention(16, 128, 0.125, 2)
    attn.k_cache, attn.v_cache = torch.zeros(2, 256, 2, 128), torch.zeros(2, 256, 2, 128)
    lens, bt = torch.tensor([7, 9], dtype=torch.int32), torch.tensor([[0], [1]], dtype=torch.int32)
    slots = torch.tensor([6, 264], dtype=torch.int32)
    k = v = torch.zeros(2, 2, 128)
    if layout == "unaligned_rows":
        k = torch.zeros(2 * 256 + 1)[1:].view(2, 2, 128)
    elif layout == "odd_row_stride":
        v = torch.zeros(2, 2 * 128 + 3)[:, :256].view(2, 2, 128)
    else:
        slots = torch.tensor([6, 264, -1], dtype=torch.int32)
    set_context(False, slot_mapping=slots, context_lens=lens, block_tables=bt)
    o = attn(torch.zeros(2, 16, 128), k, v)
    assert [c[0] for c in rec.calls] == ["store_kvcache", "flash_attn_with_kvcache"]
    assert rec.calls[0][1][0] is k and rec.calls[0][1][1] is v and rec.calls[0][1][4] is slots
    assert o == "o"


def test_decode_without_caches_calls_the_kvcache_kernel_with_an_unsqueezed_query(monkeypatch):
    rec = _Recorder(monkeypatch)
    attn = Attention(16, 128, 0.125, 2)
    lens, bt = torch.tensor([7, 9], dtype=torch.int32), torch.tensor([[0], [1]], dtype=torch.int32)
    set_context(False, slot_mapping=torch.tensor([6, 264], dtype=torch.int32), context_lens=lens, block_tables=bt)
    attn(torch.zeros(2, 16, 128), torch.zeros(2, 2, 128), torch.zeros(2, 2, 128))
    [(n1, a1, kw1)] = rec.calls
    assert n1 == "flash_attn_with_kvcache" and a1[0].shape == (2, 1, 16, 128)
    assert kw1 == dict(cache_seqlens=lens, block_table=bt, softmax_scale=0.125, causal=True)


def test_non_causal_calls_dense_attention(monkeypatch):
    rec = _Recorder(monkeypatch)
    attn = Attention(16, 128, 0.125, 2, is_causal=False)
    attn(torch.zeros(3, 5, 16, 128), torch.zeros(3, 5, 2, 128), torch.zeros(3, 5, 2, 128))
    assert [c[0] for c in rec.calls] == ["flash_attn_func"] and rec.calls[0][2] == dict(softmax_scale=0.125,
                                                                                          causal=False)


def test_context_is_read_at_call_time(monkeypatch):
    """last_rows mutates cu_seqlens_q / max_seqlen_q of the live context around one call."""
    rec = _Recorder(monkeypatch)
    attn = Attention(16, 128, 0.125, 2)
    cu = torch.tensor([0, 4, 9], dtype=torch.int32)
    set_context(True, cu, cu, 5, 5, torch.zeros(0, dtype=torch.int32), None, None)
    ctx = get_context()
    ctx.cu_seqlens_q, ctx.max_seqlen_q = torch.arange(3, dtype=torch.int32), 1
    attn(torch.zeros(2, 16, 128), torch.zeros(9, 2, 128), torch.zeros(9, 2, 128))
    kw = rec.calls[-1][2]
    assert kw["max_seqlen_q"] == 1 and kw["cu_seqlens_q"].tolist() == [0, 1, 2] and kw["cu_seqlens_k"] is cu


# --- argument checks that fire before any kernel -----------------------------------------------------------------

def test_store_kvcache_keeps_the_reference_asserts():
    from voxcpm2_arabic_dialects_turbo_amd.ops import store_kvcache

    k = torch.zeros(4, 2, 128, dtype=torch.bfloat16)
    cache = torch.zeros(2, 256, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        store_kvcache(k, k, cache, cache, torch.zeros(3, dtype=torch.int32))  # one slot per token
    with pytest.raises(AssertionError):
        store_kvcache(k.transpose(1, 2).contiguous().transpose(1, 2), k, cache, cache,
                      torch.zeros(4, dtype=torch.int32))  # last dim not contiguous
    with pytest.raises(ValueError):
        store_kvcache(k, k, cache, cache, torch.zeros(4, dtype=torch.int32))  # CPU tensors: not a GPU


def test_reference_kernel_mirrors_keep_their_contracts():
    from voxcpm2_arabic_dialects_turbo_amd.kernels.prefill_attn import paged_prefill_attention
    from voxcpm2_arabic_dialects_turbo_amd.kernels.short_attn import short_attention, short_causal_attention

    q = torch.zeros(3, 16, 128, dtype=torch.bfloat16)
    kv = torch.zeros(3, 2, 128, dtype=torch.bfloat16)
    cu = torch.tensor([0, 3], dtype=torch.int32)
    with pytest.raises(AssertionError):
        short_causal_attention(q, kv, kv, cu, 33, 0.1)  # SHORT_CAUSAL_MAX_LEN
    # the int8 modes exist; on CPU tensors they stop at the device check, before any kernel (no CPU fallback)
    with pytest.raises(ValueError, match="GPU"):
        short_causal_attention(q, kv, kv, cu, 3, 0.1, quant=True)
    with pytest.raises(ValueError, match="GPU"):
        short_attention(q.view(1, 3, 16, 128), kv.view(1, 3, 2, 128), kv.view(1, 3, 2, 128), 0.1, quant=True)
    cache = torch.zeros(2, 256, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        paged_prefill_attention(q, cache, cache, torch.zeros(1, 1, dtype=torch.int32), cu, cu, 3, 0.1, quant=True)


def test_copy_kv_block_prefix_keeps_the_reference_contract():
    """Entries with n <= 0 are dropped before anything else (no call at all); a non-contiguous cache fails the
    reference's assert; a CPU cache with work to do is rejected (no CPU fallback)."""
    from voxcpm2_arabic_dialects_turbo_amd.kernels.kv_copy import copy_kv_block_prefix

    kv = torch.zeros(2, 2, 4, 16, 2, 128, dtype=torch.bfloat16)
    copy_kv_block_prefix(kv, [(0, 1, 0), (2, 3, -5)])
    copy_kv_block_prefix(kv, [])
    with pytest.raises(AssertionError):
        copy_kv_block_prefix(kv.transpose(0, 1), [(0, 1, 3)])
    with pytest.raises(ValueError, match="GPU"):
        copy_kv_block_prefix(kv, [(0, 1, 3)])


# --- the riding stores' slot conditions (checks.py) -------------------------------------------------------------------

def _paged_step(nq, nk, bs=16, seed=3):
    """A step whose slots are the ones its tables give (disjoint blocks per sequence)."""
    gen = torch.Generator().manual_seed(seed)
    width = max((n + bs - 1) // bs for n in nk)
    perm = torch.randperm(64, generator=gen).tolist()
    tables, slots, at = torch.full((len(nk), width), -1, dtype=torch.int32), [], 0
    for b, n in enumerate(nk):
        nb = (n + bs - 1) // bs
        tables[b, :nb] = torch.tensor(perm[at:at + nb], dtype=torch.int32)
        at += nb
        slots += [int(tables[b, j // bs]) * bs + j % bs for j in range(n - nq[b], n)]
    cu = lambda x: torch.tensor([0] + torch.tensor(x).cumsum(0).tolist(), dtype=torch.int32)
    return cu(nq), cu(nk), tables, torch.tensor(slots, dtype=torch.int32)


def test_riding_store_check_passes_the_engines_slots_and_names_each_kind_of_violation():
    """The engine's slots (the tables' slots of each sequence's new positions, reference
    engine/model_runner.py:880-883 and :919) pass, prefill and decode alike; a slot that is not its table's, a new
    slot inside another sequence's context, rows missing from slot_mapping and a missing table are each reported."""
    from voxcpm2_arabic_dialects_turbo_amd.checks import riding_store_violations

    cu_q, cu_k, tables, slots = _paged_step([5, 1, 30, 1], [40, 17, 30, 3])
    kw = dict(cu_seqlens_q=cu_q, cu_seqlens_k=cu_k)
    assert riding_store_violations(slots, tables, 16, **kw) == []
    lens = torch.tensor([40, 17, 30, 3], dtype=torch.int32)
    dec = torch.tensor([int(tables[b, (n - 1) // 16]) * 16 + (n - 1) % 16 for b, n in enumerate(lens.tolist())],
                       dtype=torch.int32)
    assert riding_store_violations(dec, tables, 16, context_lens=lens) == []
    bad = slots.clone()
    bad[2] += 1  # sequence 0's third new token one slot off
    v = riding_store_violations(bad, tables, 16, **kw)
    assert len(v) == 1 and "sequence 0" in v[0] and "position 37" in v[0]
    other = slots.clone()
    other[5] = int(tables[0, 0]) * 16 + 3  # sequence 1's new token written into sequence 0's first block
    v = riding_store_violations(other, tables, 16, **kw)
    assert any("sequence 1" in m and "block table" in m for m in v)
    assert any("inside sequence 0's context" in m for m in v)
    assert "past slot_mapping" in riding_store_violations(slots[:10], tables, 16, **kw)[0]
    assert "no block tables" in riding_store_violations(slots, None, 16, **kw)[0]


def test_attention_forward_checks_the_riding_store_when_asked(monkeypatch):
    """With VOX_CHECK_STORE=1 a step whose slots break the riding store's conditions raises before any kernel runs;
    without it (the default) nothing is checked."""
    rec = _Recorder(monkeypatch)
    attn = Attention(16, 128, 0.125, 2)
    attn.k_cache, attn.v_cache = torch.zeros(64, 16, 2, 128), torch.zeros(64, 16, 2, 128)
    cu_q, cu_k, tables, slots = _paged_step([5, 1], [40, 17])
    slots[0] = -1
    set_context(True, cu_q, cu_k, 5, 40, slots, None, tables)
    q, k, v = torch.zeros(6, 16, 128), torch.zeros(6, 2, 128), torch.zeros(6, 2, 128)
    monkeypatch.setenv("VOX_CHECK_STORE", "1")
    with pytest.raises(ValueError, match="riding KV store"):
        attn(q, k, v)
    assert rec.calls == []
    monkeypatch.delenv("VOX_CHECK_STORE")
    attn(q, k, v)
    assert [c[0] for c in rec.calls] == ["prefill_attention_store"]
