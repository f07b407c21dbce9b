"""The drop-in module on the GPU: Attention.forward driven by the runner's contexts through prefill and decode steps
of a small engine loop, and the decode step captured into a HIP graph and replayed."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as ref
from tests._util import D, H, HK, attn_close, randn
from voxcpm2_arabic_dialects_turbo_amd import runner
from voxcpm2_arabic_dialects_turbo_amd.context import get_context, reset_context
from voxcpm2_arabic_dialects_turbo_amd.layers import Attention

pytestmark = pytest.mark.gpu
DEV = "cuda"
BS = 256
SCALE = D ** -0.5


@pytest.fixture(autouse=True)
def _clean_context():
    reset_context()
    yield
    reset_context()


def _model(n_layers):
    return torch.nn.ModuleList([Attention(H, D, SCALE, HK) for _ in range(n_layers)])


def _step_qkv(gen, n):
    qkv = randn(gen, n, (H + 2 * HK) * D).to(DEV)
    q, k, v = qkv.split([H * D, HK * D, HK * D], dim=-1)
    return q.view(n, H, D), k.view(n, HK, D), v.view(n, HK, D)


def _expect(layer: Attention, q, tasks, new_tokens):
    """Oracle: each sequence's query rows over its first seq_length cache slots (read back from the GPU cache)."""
    kc, vc = layer.k_cache.cpu(), layer.v_cache.cpu()
    outs, at = [], 0
    for t, n in zip(tasks, new_tokens):
        kb = ref.gather_pages(kc, t.block_table, t.seq_length).float()
        vb = ref.gather_pages(vc, t.block_table, t.seq_length).float()
        outs.append(ref.attend(q[at:at + n].float().cpu(), kb, vb, causal=True, scale=SCALE).view(n, H, D))
        at += n
    return torch.cat(outs)


def test_engine_loop_prefill_with_prefix_then_decode_steps(monkeypatch):
    """Prefill over cached prefixes (the store riding in the attention launch, tiles straddling the first new key)
    and decode steps (the store riding in the decode call) through the runner's contexts, against the oracle over the
    caches; VOX_CHECK_STORE=1 also has every step's slots checked against the riding stores' conditions."""
    monkeypatch.setenv("VOX_CHECK_STORE", "1")
    gen = torch.Generator().manual_seed(60)
    model = _model(2)
    runner.allocate_kv_cache(model, num_blocks=64, block_size=BS, device=DEV)
    for m in model:  # a reference-prefix cache: the first blocks already hold keys
        m.k_cache.copy_(randn(gen, *m.k_cache.shape).to(DEV))
        m.v_cache.copy_(randn(gen, *m.v_cache.shape).to(DEV))
    perm = torch.randperm(64, generator=gen).tolist()
    lengths, cached = [40, 300, 513, 7], [0, 260, 100, 0]
    tasks, at = [], 0
    for n, c in zip(lengths, cached):
        nb = (n + 4 + BS - 1) // BS  # room for the decode steps
        tasks.append(runner.RunnerTask(perm[at:at + nb], n, c, BS))
        at += nb
    # prefill (a cached prefix -> keys through the block tables)
    runner.prepare_prefill_context(tasks, BS, device=DEV)
    assert get_context().block_tables is not None
    new = [t.seq_length - t.num_cached_tokens for t in tasks]
    for layer in model:
        q, k, v = _step_qkv(gen, sum(new))
        o = layer(q, k, v)
        assert o.shape == (sum(new), H, D)
        attn_close(o, _expect(layer, q, tasks, new), "prefill step")
    # decode steps
    for step in range(4):
        for t in tasks:
            t.seq_length += 1
            t.num_cached_tokens = t.seq_length - 1
        runner.prepare_decode_context(tasks, BS, device=DEV)
        for layer in model:
            q, k, v = _step_qkv(gen, len(tasks))
            o = layer(q, k, v)
            assert o.shape == (len(tasks), 1, H, D)
            attn_close(o[:, 0], _expect(layer, q, tasks, [1] * len(tasks)), f"decode step {step}")


def test_decode_step_captured_in_a_graph_replays_like_eager():
    """Static buffers + torch.cuda.graph, as the reference's capture_cudagraph: warm-up eager call, capture, then
    several replays with eager work and synchronizations between them, each checked against an eager run."""
    gen = torch.Generator().manual_seed(61)
    model = _model(3)
    runner.allocate_kv_cache(model, num_blocks=64, block_size=BS, device=DEV)
    for m in model:
        m.k_cache.copy_(randn(gen, *m.k_cache.shape).to(DEV))
        m.v_cache.copy_(randn(gen, *m.v_cache.shape).to(DEV))
    max_bs, max_blocks = 16, 4
    bufs = runner.DecodeGraphBuffers(max_bs, max_blocks, device=DEV)
    q_in = torch.zeros(max_bs, (H + 2 * HK) * D, dtype=torch.bfloat16, device=DEV)
    out = torch.zeros(3, max_bs, H * D, dtype=torch.bfloat16, device=DEV)

    def forward(bs):
        qkv = q_in[:bs]
        q, k, v = qkv.split([H * D, HK * D, HK * D], dim=-1)
        for i, layer in enumerate(model):
            out[i, :bs] = layer(q.view(bs, H, D), k.view(bs, HK, D), v.view(bs, HK, D)).view(bs, -1)

    bs = 16
    bufs.bind(bs)
    forward(bs)  # warm-up (context_lens all zero)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        forward(bs)
    perm = torch.randperm(64, generator=gen).tolist()  # sequence i owns blocks perm[4i : 4i + 4]
    for rep in range(4):
        n = [16, 9, 16, 5][rep]
        tasks = []
        for i in range(n):
            length = int(torch.randint(1, max_blocks * BS + 1, (1,), generator=gen))
            nb = (length + BS - 1) // BS
            tasks.append(runner.RunnerTask(perm[4 * i:4 * i + nb], length, length - 1, BS))
        q_in[:n].copy_(randn(gen, n, (H + 2 * HK) * D).to(DEV))
        runner.prepare_decode_context(tasks, BS, device=DEV)
        bufs.load()
        bufs.bind(bs)
        graph.replay()
        torch.cuda.synchronize()
        replayed = out[:, :n].clone()
        runner.prepare_decode_context(tasks, BS, device=DEV)  # eager run of the same step
        forward(n)
        torch.cuda.synchronize()
        assert torch.equal(replayed, out[:, :n]), f"replay {rep} differs from eager"
        for i, layer in enumerate(model):
            q = q_in[:n, :H * D].view(n, H, D)
            attn_close(out[i, :n].view(n, H, D), _expect(layer, q, tasks, [1] * n), f"replay {rep} layer {i}")


@pytest.mark.parametrize("cached", [[0, 0, 0, 0], [0, 260, 100, 3]])
def test_last_rows_through_attention_forward(cached):
    """The residual LM's last layer (reference: kernels/fused_layer.py:749-781) through Attention.forward: the KV
    store inside uses every row of the step (slot_mapping unchanged), while cu_seqlens_q = arange(n + 1) and
    max_seqlen_q = 1 are set in place on the live context for the one call, with the last row of each sequence as
    its query. Without a cached prefix the keys are the step's own rows; with one, they come through the tables."""
    gen = torch.Generator().manual_seed(64 + sum(cached))
    layer = Attention(H, D, SCALE, HK)
    runner.allocate_kv_cache([layer], num_blocks=32, block_size=BS, device=DEV)
    layer.k_cache.copy_(randn(gen, *layer.k_cache.shape).to(DEV))
    layer.v_cache.copy_(randn(gen, *layer.v_cache.shape).to(DEV))
    perm = torch.randperm(32, generator=gen).tolist()
    lengths = [40, 300, 513, 7]
    tasks, at = [], 0
    for n, c in zip(lengths, cached):
        nb = (n + BS - 1) // BS
        tasks.append(runner.RunnerTask(perm[at:at + nb], n, c, BS))
        at += nb
    new = [n - c for n, c in zip(lengths, cached)]
    T = sum(new)
    runner.prepare_prefill_context(tasks, BS, device=DEV)
    q, k, v = _step_qkv(gen, T)
    rows = torch.tensor(np.cumsum(new) - 1, device=DEV)
    ctx = get_context()
    saved = ctx.cu_seqlens_q, ctx.max_seqlen_q
    ctx.cu_seqlens_q, ctx.max_seqlen_q = torch.arange(len(tasks) + 1, dtype=torch.int32, device=DEV), 1
    try:
        o = layer(q[rows].contiguous(), k, v)
    finally:
        ctx.cu_seqlens_q, ctx.max_seqlen_q = saved
    torch.cuda.synchronize()
    assert o.shape == (len(tasks), H, D)
    # every row's K/V went to its slot; the last row of each sequence attends over the sequence's whole length
    want = _expect(layer, q[rows], tasks, [1] * len(tasks))
    attn_close(o, want, f"last rows, cached {cached}")
    kc = layer.k_cache.cpu()
    at = 0
    for t, n in zip(tasks, new):
        got_rows = torch.stack([kc.view(-1, HK, D)[ref.slot_of(t.block_table, j, BS)]
                                for j in range(t.num_cached_tokens, t.seq_length)])
        assert torch.equal(got_rows, k[at:at + n].cpu()), "the store must write every row of the step"
        at += n
