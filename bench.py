#!/usr/bin/env python
"""Benchmark of the paged-KV attention path on one MI355X.

Headline (``value``): benchmark config 4, paged decode at peak concurrency across a 28-layer stack. One step = the 28
layers' ``Attention.forward`` decode calls (KV store of the new token + split-KV paged decode) for 150 sequences
with contexts U[256, 2048], 16 query / 2 KV heads, head_dim 128, bf16, 256-token blocks; each layer has its own
[2048, 256, 2, 128] K and V planes and its own q, seeded independently; the block tables (non-overlapping ids from a
shuffled 2048-block pool) are shared by the layers, as an engine's are. The step is captured into a HIP graph and
replayed, as the reference engine runs its decode step. ``value`` = algorithmic bytes of the step / step time.

Beside it: the decode kernel's roofline (average launch duration from a graph of the 28 decode launches, HIP
events on the launch stream), the prefill metric on benchmark config 2 (varlen causal prefill, TFLOP/s against the
bf16 dense MFMA peak, inputs rotated through > 256 MB so the Infinity Cache cannot serve them) plus a compute-bound
supplementary prefill shape, and the CPU baseline: the oracle's torch path on the host cores over a bounded sample of
the same decode workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--decode-only]
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E, GB/s
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, TFLOP/s
H, HK, D, BS = 16, 2, 128, 256
SCALE = D ** -0.5


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle timing")
    p.add_argument("--decode-only", action="store_true", help="headline decode only (no prefill legs)")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline sample budget")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="also run 5 device copies of 256 MiB: the reference a PMC byte counter is scaled by")
    return p.parse_args()


# ---------------------------------------------------------------------------------------------------------------------

def _graph_ms(fn, reps: int, warm: int = 3, warm_s: float = 0.15) -> float:
    """Captures fn() in a HIP graph (after one eager warm-up call) and returns ms per replay over `reps` replays,
    timed by HIP events on the current stream. The untimed warm-up replays run for at least `warm_s` seconds (and
    `warm` replays): the GPU's clocks take some 0.1 s of sustained load to settle, and a leg timed straight after a
    lighter one reads up to 25 % slow (16 x 2048 prefill: 361 -> 279 us over its first ~0.1 s)."""
    import torch

    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    t0, n = time.perf_counter(), 0
    while n < warm or time.perf_counter() - t0 < warm_s:
        g.replay()
        torch.cuda.synchronize()
        n += 1
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        g.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / reps


def decode_bytes(lens) -> int:
    """Algorithmic HBM bytes of one decode launch: K+V of every context token, q and o, context_lens and the block
    table entries read."""
    toks = sum(lens)
    blocks = sum((n + BS - 1) // BS for n in lens)
    return toks * HK * D * 2 * 2 + len(lens) * H * D * 2 * 2 + 4 * (len(lens) + blocks)


def store_bytes(n: int) -> int:
    """Algorithmic bytes of storing n tokens' K/V rows: read k and v rows, write them, read the slots."""
    return n * HK * D * 2 * 2 * 2 + 4 * n


def prefill_units(nq, nk):
    """(flops, bytes) of a varlen causal prefill: QK^T and PV over unmasked pairs; q, o and the K/V read once."""
    pairs = sum(sum(k - q + i + 1 for i in range(q)) for q, k in zip(nq, nk))
    flops = 4 * D * H * pairs
    nbytes = sum(nq) * H * D * 2 * 2 + sum(nk) * HK * D * 2 * 2
    return flops, nbytes


# ---------------------------------------------------------------------------------------------------------------------

class DecodeWorkload:
    """Benchmark config 4: 150 sequences x 28 layers, contexts U[256, 2048]."""

    B, LAYERS, POOL = 150, 28, 2048

    def __init__(self, dev):
        import torch

        from voxcpm2_arabic_dialects_turbo_amd import runner
        from voxcpm2_arabic_dialects_turbo_amd.layers import Attention

        gen = torch.Generator().manual_seed(100)
        self.lens = torch.randint(256, 2049, (self.B,), generator=gen).tolist()
        perm = torch.randperm(self.POOL, generator=gen).tolist()
        tasks, at = [], 0
        for n in self.lens:
            nb = (n + BS - 1) // BS
            tasks.append(runner.RunnerTask(perm[at:at + nb], n, n - 1, BS))
            at += nb
        self.tasks = tasks
        self.layers = [Attention(H, D, SCALE, HK) for _ in range(self.LAYERS)]
        self.kv = runner.allocate_kv_cache(self.layers, num_blocks=self.POOL, block_size=BS, device=dev)
        self.qkv = torch.empty(self.LAYERS, self.B, (H + 2 * HK) * D, dtype=torch.bfloat16, device=dev)
        for i in range(self.LAYERS):
            g = torch.Generator(device=dev).manual_seed(100 + i)
            self.kv[i].normal_(generator=g)
            self.qkv[i].normal_(generator=g)
        self.out = torch.empty(self.LAYERS, self.B, H * D, dtype=torch.bfloat16, device=dev)
        runner.prepare_decode_context(tasks, BS, device=dev)
        torch.cuda.synchronize()

    def views(self, i):
        q, k, v = self.qkv[i].split([H * D, HK * D, HK * D], dim=-1)
        return q.view(self.B, H, D), k.view(self.B, HK, D), v.view(self.B, HK, D)

    def step(self):
        """One decode step: every layer's Attention.forward (store + decode). The outputs are left where the call
        allocated them (the caller only views them: reference nanovllm_voxcpm/model/model.py:224-226)."""
        outs = []
        for i, layer in enumerate(self.layers):
            q, k, v = self.views(i)
            outs.append(layer(q, k, v))
        return outs

    def decode_launches(self):
        """The step's 28 decode-kernel launches alone (no store), for the kernel's roofline; planned as a step's
        layers are (the first call records the layout, the others reuse it)."""
        from voxcpm2_arabic_dialects_turbo_amd.context import get_context
        from voxcpm2_arabic_dialects_turbo_amd.ops import decode_attention

        ctx = get_context()
        for i, layer in enumerate(self.layers):
            q, _, _ = self.views(i)
            decode_attention(q, layer.k_cache, layer.v_cache, ctx.context_lens, ctx.block_tables, SCALE,
                             out=self.out[i].view(self.B, H, D), plan=("bench decode launches", id(ctx)))

    def step_bytes(self) -> int:
        return self.LAYERS * (decode_bytes(self.lens) + store_bytes(self.B))


def bench_decode(args, dev):
    import torch

    w = DecodeWorkload(dev)
    # full step in a graph (what `value` measures)
    w.step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        w.step()
    for _ in range(args.warmup):
        g.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        g.replay()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(stop) / args.steps
    # the decode kernel alone: graph of its 28 launches, HIP events on the launch stream
    reps = max(10, args.steps // 2)
    per_launch_ms = _graph_ms(w.decode_launches, reps) / w.LAYERS
    res = dict(ms_per_step=ms_per_step, wall_s=wall, step_bytes=w.step_bytes(),
               launch_bytes=decode_bytes(w.lens), launch_ms=per_launch_ms, lens=w.lens, workload=w)
    return res


def _rand_bf16(shape, seed, dev):
    import torch

    return torch.randn(*shape, generator=torch.Generator(device=dev).manual_seed(seed), device=dev).to(torch.bfloat16)


def bench_config3(dev):
    """Benchmark config 3: one decode call over 40 sequences, contexts U[200, 1500], each input set with its own
    1024-block pool (bf16 K and V planes of [1024, 256, 2, 128]) and block tables of non-overlapping ids from a
    shuffled pool; 10 sets (>= 350 MB read per rotation) so the Infinity Cache cannot serve them."""
    import torch

    from voxcpm2_arabic_dialects_turbo_amd.ops import decode_attention

    B, POOL, SETS = 40, 1024, 10
    gen = torch.Generator().manual_seed(30)
    lens = torch.randint(200, 1501, (B,), generator=gen).tolist()
    width = max((n + BS - 1) // BS for n in lens)
    tables = []
    for _ in range(SETS):
        perm = torch.randperm(POOL, generator=gen).tolist()
        t, at = torch.full((B, width), -1, dtype=torch.int32), 0
        for b, n in enumerate(lens):
            nb = (n + BS - 1) // BS
            t[b, :nb] = torch.tensor(perm[at:at + nb], dtype=torch.int32)
            at += nb
        tables.append(t.to(dev))
    kv = _rand_bf16((SETS, 2, POOL, BS, HK, D), 31, dev)
    q = _rand_bf16((SETS, B, H, D), 32, dev)
    lens_d = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = torch.empty(B, H, D, dtype=torch.bfloat16, device=dev)

    def run():
        for i in range(SETS):
            decode_attention(q[i], kv[i, 0], kv[i, 1], lens_d, tables[i], SCALE, out=out)

    ms = _graph_ms(run, 20) / SETS
    nbytes = decode_bytes(lens)
    gbs = nbytes / (ms * 1e-3) / 1e9

    # the same call as a layer of a decode step: 28 layers over one set of lengths and tables (each layer its own
    # K/V planes and q, cycling over the 10 sets' planes: > 256 MB between two reads of one plane); the first layer
    # records the layout, the others reuse it, as Attention.forward plans a step
    LAYERS = 28

    def run_step():
        for i in range(LAYERS):
            s = i % SETS
            decode_attention(q[s], kv[s, 0], kv[s, 1], lens_d, tables[0], SCALE, out=out, plan=("bench config 3",))

    ms_step = _graph_ms(run_step, 20) / LAYERS
    del kv
    return dict(workload="BASELINE config 3: decode, 40 seqs, ctx U[200,1500], 1024-block pool, one layer",
                launch_us=round(ms * 1e3, 2), launch_bytes=nbytes, gbs=round(gbs, 1),
                frac_hbm_peak=round(gbs / HBM_PEAK_GBS, 4), input_sets=SETS,
                launch_us_in_step=round(ms_step * 1e3, 2),
                in_step_what="the same call as one of 28 layers of a decode step sharing lengths and tables "
                             "(layout recorded by the first layer, reused by the others)")


def bench_config5(dev):
    """Benchmark config 5: a mixed chunked-prefill + decode step in one varlen paged call. 6 new prefills of U[300,
    600] tokens (no cached prefix) and 120 decode rows (one new token over U[128, 1800] cached ones), in the
    scheduler's order (prefills, then the decode riders); the step's new K/V rows (every prefill token and each
    decode row's token) are stored first through store_kvcache, as Attention.forward does. 2048-block pool (bf16 K and
    V planes [2048, 256, 2, 128]); 3 input sets on disjoint blocks (>= 440 MB read per rotation). Reports the step
    (store + attention, Attention.forward) and the attention launch alone against its roofline
    max(bytes / HBM peak, flops / MFMA peak)."""
    import torch

    from voxcpm2_arabic_dialects_turbo_amd.context import reset_context, set_context
    from voxcpm2_arabic_dialects_turbo_amd.layers import Attention
    from voxcpm2_arabic_dialects_turbo_amd.ops import varlen_attention

    POOL, SETS = 2048, 3
    gen = torch.Generator().manual_seed(51)
    pre = torch.randint(300, 601, (6,), generator=gen).tolist()
    dec = torch.randint(128, 1801, (120,), generator=gen).tolist()
    nk = pre + dec
    nq = pre + [1] * len(dec)
    width = max((n + BS - 1) // BS for n in nk)
    perm = torch.randperm(POOL, generator=gen).tolist()
    tables, slots, at = [], [], 0
    for _ in range(SETS):
        t = torch.full((len(nk), width), -1, dtype=torch.int32)
        sl = []
        for b, n in enumerate(nk):
            nb = (n + BS - 1) // BS
            ids = perm[at:at + nb]
            at += nb
            t[b, :nb] = torch.tensor(ids, dtype=torch.int32)
            sl += [ids[j // BS] * BS + j % BS for j in range(n - nq[b], n)]
        tables.append(t.to(dev))
        slots.append(torch.tensor(sl, dtype=torch.int32, device=dev))
    assert at <= POOL
    T = sum(nq)
    layer = Attention(H, D, SCALE, HK)
    kv = _rand_bf16((2, POOL, BS, HK, D), 52, dev)
    layer.k_cache, layer.v_cache = kv[0], kv[1]
    qkv = _rand_bf16((SETS, T, (H + 2 * HK) * D), 53, dev)
    cu_q = torch.tensor([0] + torch.tensor(nq).cumsum(0).tolist(), dtype=torch.int32, device=dev)
    cu_k = torch.tensor([0] + torch.tensor(nk).cumsum(0).tolist(), dtype=torch.int32, device=dev)
    o = torch.empty(T, H, D, dtype=torch.bfloat16, device=dev)

    def views(i):
        q, k, v = qkv[i].split([H * D, HK * D, HK * D], dim=-1)
        return q.view(T, H, D), k.view(T, HK, D), v.view(T, HK, D)

    def run_step():
        for i in range(SETS):
            set_context(True, cu_q, cu_k, max(nq), max(nk), slots[i], None, tables[i])
            q, k, v = views(i)
            layer(q, k, v)

    def run_attn():
        for i in range(SETS):
            varlen_attention(views(i)[0], None, None, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=max(nq),
                             softmax_scale=SCALE, causal=True, block_table=tables[i], k_cache=kv[0], v_cache=kv[1],
                             out=o)

    try:
        step_ms = _graph_ms(run_step, 20) / SETS
    finally:
        reset_context()
    ms = _graph_ms(run_attn, 20) / SETS
    flops, nbytes = prefill_units(nq, nk)
    t_roof = max(nbytes / (HBM_PEAK_GBS * 1e9), flops / (MFMA_BF16_PEAK_TFLOPS * 1e12))
    del kv, qkv
    return dict(workload="BASELINE config 5: one varlen paged call, 6 prefills U[300,600] + 120 decode rows "
                         "ctx U[128,1800], 2048-block pool",
                step_us=round(step_ms * 1e3, 2), launch_us=round(ms * 1e3, 2), flops=flops, bytes=nbytes,
                tflops=round(flops / (ms * 1e-3) / 1e12, 2), gbs=round(nbytes / (ms * 1e-3) / 1e9, 1),
                pct_mfma_peak=round(100 * flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 2),
                pct_hbm_peak=round(100 * nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                roofline_us=round(t_roof * 1e6, 2), frac_of_roofline=round(t_roof / (ms * 1e-3), 4),
                bound="hbm" if nbytes / (HBM_PEAK_GBS * 1e9) >= flops / (MFMA_BF16_PEAK_TFLOPS * 1e12) else "mfma",
                input_sets=SETS)


def bench_ceiling(dev, w):
    """What the HBM path delivers to loads alone, measured in this run (libvoxprobe.so): a grid-stride read of
    169.6 MB regions of a 1.2 GB buffer (rotating, so the Infinity Cache cannot serve them), and the decode kernel's
    own loads on the config-4 workload (same tiles, same per-wave load layout, same equal contiguous ranges over 256
    workgroups, rotating over the 28 layers' planes) without its arithmetic."""
    import ctypes

    import numpy as np
    import torch

    from voxcpm2_arabic_dialects_turbo_amd import _lib

    probe = ctypes.CDLL(os.path.join(ROOT, "voxcpm2_arabic_dialects_turbo_amd", "libvoxprobe.so"))
    probe.vox_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                            ctypes.c_void_p]
    probe.vox_probe_tile_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                          ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    sink = torch.empty(1024, dtype=torch.uint8, device=dev)
    region = decode_bytes(w.lens) // 4096 * 4096
    regions = 14  # 2.4 GB: neither one region nor the rotation fits the 256 MB Infinity Cache
    buf = torch.empty(region * regions, dtype=torch.uint8, device=dev)
    buf.fill_(1)
    out = {"stream_read": {}, "decode_pattern_read": {}}
    for grid in (256, 1024, 2048):
        # 28 back-to-back launches of one layer's bytes (as many as a decode step has calls), rotating regions
        def run(grid=grid):
            for r in range(w.LAYERS):
                assert probe.vox_probe_stream_read(buf.data_ptr() + (r % regions) * region, region, sink.data_ptr(),
                                                   grid, _lib.stream_handle(dev)) == 0

        ms = _graph_ms(run, 10) / w.LAYERS
        out["stream_read"][f"grid{grid}"] = round(region / (ms * 1e-3) / 1e9, 1)
    out["stream_read_launch_bytes"] = region
    # the sustained rate: one launch over the whole 2.4 GB, so its start and end cost little against its length;
    # what separates it from the per-layer launches above is each launch's ramp and tail
    sustained = {}
    for grid in (1024, 2048, 4096):
        def run_all(grid=grid):
            assert probe.vox_probe_stream_read(buf.data_ptr(), region * regions, sink.data_ptr(), grid,
                                               _lib.stream_handle(dev)) == 0

        ms = _graph_ms(run_all, 5)
        sustained[f"grid{grid}"] = round(region * regions / (ms * 1e-3) / 1e9, 1)
    out["stream_read_sustained"] = sustained
    out["stream_read_sustained_bytes"] = region * regions
    out["stream_read_sustained_gbs"] = max(sustained.values())
    del buf
    # tile offsets of the decode workload: 16-token tiles of every sequence, sequence by sequence
    offs = []
    for t in w.tasks:
        for tok in range(0, t.seq_length, 16):
            offs.append((t.block_table[tok // BS] * BS + tok % BS) * HK * D * 2)
    tiles = torch.tensor(np.asarray(offs, dtype=np.int64), device=dev)
    tile_bytes = len(offs) * 16 * HK * D * 2 * 2
    for grid, depth in ((256, 1), (256, 2), (512, 1), (512, 2)):
        def run(grid=grid, depth=depth):
            for i, layer in enumerate(w.layers):
                assert probe.vox_probe_tile_read(layer.k_cache.data_ptr(), layer.v_cache.data_ptr(),
                                                 tiles.data_ptr(), len(offs), sink.data_ptr(), grid, depth,
                                                 _lib.stream_handle(dev)) == 0

        ms = _graph_ms(run, 10) / len(w.layers)
        out["decode_pattern_read"][f"grid{grid}_depth{depth}"] = round(tile_bytes / (ms * 1e-3) / 1e9, 1)
    out["stream_read_best_gbs"] = max(out["stream_read"].values())
    out["decode_pattern_read_best_gbs"] = max(out["decode_pattern_read"].values())
    out["decode_pattern_bytes"] = tile_bytes
    return out


def bench_prefill(dev):
    """Benchmark config 2 prefill (packed causal varlen, production's no-prefix path) and a supplementary
    compute-bound shape; per-launch ms from graphs of launches rotating over input sets."""
    import torch

    from voxcpm2_arabic_dialects_turbo_amd.ops import varlen_attention

    out = {}
    gen = torch.Generator().manual_seed(50)
    lens = torch.randint(64, 513, (8,), generator=gen).tolist()
    T = sum(lens)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=dev)
    set_bytes = T * (H + 2 * HK) * D * 2
    n_sets = max(2, (300 << 20) // set_bytes + 1)  # > 256 MB of inputs: not served from the Infinity Cache
    qkv = torch.randn(n_sets, T, (H + 2 * HK) * D, generator=torch.Generator(device=dev).manual_seed(50),
                      device=dev).to(torch.bfloat16)
    o = torch.empty(T, H, D, dtype=torch.bfloat16, device=dev)

    def run_c2():
        for s in range(n_sets):
            q, k, v = qkv[s].split([H * D, HK * D, HK * D], dim=-1)
            varlen_attention(q.view(T, H, D), k.view(T, HK, D), v.view(T, HK, D), cu_seqlens_q=cu, cu_seqlens_k=cu,
                             max_seqlen_q=max(lens), softmax_scale=SCALE, causal=True, out=o)

    ms = _graph_ms(run_c2, 20) / n_sets
    flops, nbytes = prefill_units(lens, lens)
    tf = flops / (ms * 1e-3) / 1e12
    bound = min(MFMA_BF16_PEAK_TFLOPS, flops / nbytes * HBM_PEAK_GBS / 1e3)
    out["config2"] = dict(lens=lens, tokens=T, launch_us=round(ms * 1e3, 2), tflops=round(tf, 2),
                          pct_mfma_peak=round(100 * tf / MFMA_BF16_PEAK_TFLOPS, 2),
                          flop_per_byte=round(flops / nbytes, 1), roofline_bound_tflops=round(bound, 1),
                          pct_of_roofline_bound=round(100 * tf / bound, 2), input_sets=n_sets)
    # the same launches with the int8 output epilogue (o * inv_smooth -> int8 + per-token scale, the W8A8 o_proj's
    # input); the output bytes shrink to T x (H x D + 4)
    inv_smooth = torch.rand(H * D, generator=torch.Generator(device=dev).manual_seed(52), device=dev) + 0.5

    def run_c2_int8():
        for s in range(n_sets):
            q, k, v = qkv[s].split([H * D, HK * D, HK * D], dim=-1)
            varlen_attention(q.view(T, H, D), k.view(T, HK, D), v.view(T, HK, D), cu_seqlens_q=cu, cu_seqlens_k=cu,
                             max_seqlen_q=max(lens), softmax_scale=SCALE, causal=True, quant=True,
                             inv_smooth=inv_smooth)

    ms8 = _graph_ms(run_c2_int8, 20) / n_sets
    tf8 = flops / (ms8 * 1e-3) / 1e12
    out["config2_int8_output"] = dict(launch_us=round(ms8 * 1e3, 2), tflops=round(tf8, 2),
                                      pct_mfma_peak=round(100 * tf8 / MFMA_BF16_PEAK_TFLOPS, 2))
    # the same step in paged mode (the configuration's other mode): keys and values read through the block tables
    # from 256-token blocks of a 512-block pool (3 pools with shuffled tables, 403 MB; the queries from the packed
    # leg's 30 sets)
    POOL, PSETS = 512, 3
    kvp = _rand_bf16((PSETS, 2, POOL, BS, HK, D), 53, dev)
    ptables = []
    pgen = torch.Generator().manual_seed(54)
    width = max((n + BS - 1) // BS for n in lens)
    for _ in range(PSETS):
        perm, at = torch.randperm(POOL, generator=pgen).tolist(), 0
        t = torch.full((len(lens), width), -1, dtype=torch.int32)
        for b, n in enumerate(lens):
            nb = (n + BS - 1) // BS
            t[b, :nb] = torch.tensor(perm[at:at + nb], dtype=torch.int32)
            at += nb
        ptables.append(t.to(dev))

    PREPS = 10  # the sets 10 times over in one graph: 30 launches, as many as the packed leg's, so the graph's own
                # launch cost weighs the same per launch

    def run_c2_paged():
        for i in range(PSETS * PREPS):
            s = i % PSETS
            q = qkv[i % n_sets][:, :H * D].view(T, H, D)
            varlen_attention(q, None, None, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens),
                             softmax_scale=SCALE, causal=True, block_table=ptables[s], k_cache=kvp[s, 0],
                             v_cache=kvp[s, 1], out=o)

    msp = _graph_ms(run_c2_paged, 20) / (PSETS * PREPS)
    tfp = flops / (msp * 1e-3) / 1e12
    out["config2_paged"] = dict(launch_us=round(msp * 1e3, 2), tflops=round(tfp, 2),
                                pct_mfma_peak=round(100 * tfp / MFMA_BF16_PEAK_TFLOPS, 2), input_sets=PSETS)
    # the whole config-2 step as BASELINE defines it: Attention.forward stores the step's K/V rows at their slots
    # (256-token blocks of the shuffled pool) and then attends, over the packed rows (no cached prefix: block_tables
    # None) or through the block tables (prefix-cache mode, the keys read back from the pool just written);
    # reference nanovllm_voxcpm/model/layers.py:332-348
    from voxcpm2_arabic_dialects_turbo_amd.context import reset_context, set_context
    from voxcpm2_arabic_dialects_turbo_amd.layers import Attention

    layer = Attention(H, D, SCALE, HK)
    pslots = []
    for s in range(PSETS):
        tb = ptables[s].cpu()
        pslots.append(torch.tensor([int(tb[b, j // BS]) * BS + j % BS for b, n in enumerate(lens) for j in range(n)],
                                   dtype=torch.int32, device=dev))

    def run_c2_step(paged):
        def fn():
            for i in range(PSETS * PREPS):
                s = i % PSETS
                layer.k_cache, layer.v_cache = kvp[s, 0], kvp[s, 1]
                set_context(True, cu, cu, max(lens), max(lens), pslots[s], None, ptables[s] if paged else None)
                q, k, v = qkv[i % n_sets].split([H * D, HK * D, HK * D], dim=-1)
                layer(q.view(T, H, D), k.view(T, HK, D), v.view(T, HK, D))
        return fn

    try:
        for key, paged in (("config2", False), ("config2_paged", True)):
            mss = _graph_ms(run_c2_step(paged), 20) / (PSETS * PREPS)
            out[key]["step_us"] = round(mss * 1e3, 2)
            out[key]["step_what"] = ("Attention.forward: store_kvcache of the step's K/V rows, then the varlen "
                                     "causal prefill " + ("through the block tables" if paged else
                                                          "over the packed rows"))
    finally:
        reset_context()
    del qkv, kvp
    # supplementary compute-bound shape: 16 sequences x 2048 tokens, causal
    L, NB = 2048, 16
    T2 = L * NB
    big = torch.randn(T2, (H + 2 * HK) * D, generator=torch.Generator(device=dev).manual_seed(51),
                      device=dev).to(torch.bfloat16)
    cu2 = torch.arange(0, T2 + 1, L, dtype=torch.int32, device=dev)
    o2 = torch.empty(T2, H, D, dtype=torch.bfloat16, device=dev)
    q, k, v = big.split([H * D, HK * D, HK * D], dim=-1)

    def run_long():
        varlen_attention(q.view(T2, H, D), k.view(T2, HK, D), v.view(T2, HK, D), cu_seqlens_q=cu2, cu_seqlens_k=cu2,
                         max_seqlen_q=L, softmax_scale=SCALE, causal=True, out=o2)

    ms2 = _graph_ms(run_long, 10)
    flops2, _ = prefill_units([L] * NB, [L] * NB)
    tf2 = flops2 / (ms2 * 1e-3) / 1e12
    out["long_16x2048_supplementary"] = dict(launch_us=round(ms2 * 1e3, 1), tflops=round(tf2, 1),
                                             pct_mfma_peak=round(100 * tf2 / MFMA_BF16_PEAK_TFLOPS, 2))
    del big, o2
    out["chain_latency"] = bench_chain_latency(dev)
    return out


def bench_chain_latency(dev, sets: int = 32):
    """Launch time of one causal sequence of n tokens, for growing n: the sequence's heaviest work item (its last q
    tile) walks ceil(n / 64) key tiles one after another, and the light items run beside it, so the launch time
    against that count gives the fixed start and the cost per key tile of a chain (what bounds config 2). Inputs
    rotate over `sets` copies per length."""
    import torch

    from voxcpm2_arabic_dialects_turbo_amd.ops import varlen_attention

    rows, xs, ys = [], [], []
    for n in (64, 128, 256, 512, 1024):
        buf = torch.randn(sets, n, (H + 2 * HK) * D, generator=torch.Generator(device=dev).manual_seed(52),
                          device=dev).to(torch.bfloat16)
        cu1 = torch.tensor([0, n], dtype=torch.int32, device=dev)
        o1 = torch.empty(n, H, D, dtype=torch.bfloat16, device=dev)

        def run():
            for s in range(sets):
                q, k, v = buf[s].split([H * D, HK * D, HK * D], dim=-1)
                varlen_attention(q.view(n, H, D), k.view(n, HK, D), v.view(n, HK, D), cu_seqlens_q=cu1,
                                 cu_seqlens_k=cu1, max_seqlen_q=n, softmax_scale=SCALE, causal=True, out=o1)

        us = _graph_ms(run, 20) / sets * 1e3
        tiles = (n + 63) // 64
        rows.append(dict(tokens=n, key_tiles_of_heaviest_item=tiles, launch_us=round(us, 2)))
        xs.append(tiles)
        ys.append(us)
        del buf, o1
    mx, my = sum(xs) / len(xs), sum(ys) / len(ys)
    slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
    return dict(what="one causal sequence per launch (16 q / 2 kv heads), launch time by length", runs=rows,
                fit_us_per_key_tile=round(slope, 3), fit_start_us=round(my - slope * mx, 2))


def bench_reference_shapes(dev):
    """The workloads the reference publishes per-layer GPU times for (nanovllm_voxcpm/kernels/prefill_attn.py:10-12,
    kernels/short_attn.py:159-161; measured there on an NVIDIA A10): paged causal prefill of 44 sequences x 46 new
    tokens over a 50-token cached prefix (bf16 output, and the fused int8 output), and the head-start step of 200
    sequences x 7 tokens with no prefix. Inputs rotate through > 256 MB so the Infinity Cache cannot serve them; the
    published reference figures ride along for comparison (different hardware)."""
    import torch

    from voxcpm2_arabic_dialects_turbo_amd.ops import varlen_attention

    out = {}
    # 44 x 46 new tokens over a 50-token prefix, paged (256-token blocks, one block per sequence)
    B, NEW, PRE = 44, 46, 50
    nk = NEW + PRE
    gq = torch.Generator(device=dev).manual_seed(60)
    set_bytes = B * NEW * H * D * 2 + B * BS * HK * D * 2 * 2
    n_sets = max(2, (300 << 20) // set_bytes + 1)
    pool = n_sets * B
    kc = torch.randn(pool, BS, HK, D, generator=gq, device=dev).to(torch.bfloat16)
    vc = torch.randn(pool, BS, HK, D, generator=gq, device=dev).to(torch.bfloat16)
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(61)).to(torch.int32)
    tables = perm.view(n_sets, B, 1).to(dev)
    qs = torch.randn(n_sets, B * NEW, H, D, generator=gq, device=dev).to(torch.bfloat16)
    cu_q = torch.arange(0, B * NEW + 1, NEW, dtype=torch.int32, device=dev)
    cu_k = torch.arange(0, B * nk + 1, nk, dtype=torch.int32, device=dev)
    o = torch.empty(B * NEW, H, D, dtype=torch.bfloat16, device=dev)

    def run_paged(quant):
        def fn():
            for i in range(n_sets):
                varlen_attention(qs[i], None, None, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=NEW,
                                 softmax_scale=SCALE, causal=True, block_table=tables[i], k_cache=kc, v_cache=vc,
                                 out=None if quant else o, quant=quant)
        return fn

    for quant, key, ref in ((False, "paged_prefill_44x46_prefix50", {"fa2_a10_us": "70-76"}),
                            (True, "paged_prefill_44x46_prefix50_int8", {"fa2_plus_quant_a10_us": 103,
                                                                        "triton_fused_int8_a10_us": "66-74"})):
        ms = _graph_ms(run_paged(quant), 20) / n_sets
        flops, nbytes = prefill_units([NEW] * B, [nk] * B)
        out[key] = dict(launch_us=round(ms * 1e3, 2), tflops=round(flops / (ms * 1e-3) / 1e12, 2),
                        reference_published=ref)
    # the same steps with their KV store (the 46 new tokens at positions 50-95 of each sequence's block): the store
    # riding in the attention launch (prefill_attention_store with the block table; int8: the W8A8 layer's
    # store_kvcache + paged_prefill_attention pair, kernels/fused_layer.py:619-641) against the two calls
    from voxcpm2_arabic_dialects_turbo_amd.ops import prefill_attention_store, store_kvcache

    pos = torch.arange(PRE, nk, device=dev).repeat(B)
    pslots = [(tables[i].view(-1).long().repeat_interleave(NEW) * BS + pos).to(torch.int32) for i in range(n_sets)]
    kvr = torch.randn(n_sets, 2, B * NEW, HK, D, generator=gq, device=dev).to(torch.bfloat16)
    inv = torch.rand(H * D, generator=gq, device=dev) + 0.5

    def run_paged_step(quant, riding):
        def fn():
            for i in range(n_sets):
                kw = dict(cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=NEW, softmax_scale=SCALE, causal=True,
                          block_table=tables[i], quant=quant, inv_smooth=inv if quant else None)
                if riding:
                    prefill_attention_store(qs[i], kvr[i, 0], kvr[i, 1], kc, vc, pslots[i], **kw)
                else:
                    store_kvcache(kvr[i, 0], kvr[i, 1], kc, vc, pslots[i])
                    varlen_attention(qs[i], None, None, k_cache=kc, v_cache=vc, **kw)
        return fn

    for quant, key in ((False, "paged_prefill_44x46_prefix50"), (True, "paged_prefill_44x46_prefix50_int8")):
        step = _graph_ms(run_paged_step(quant, True), 20) / n_sets
        two = _graph_ms(run_paged_step(quant, False), 20) / n_sets
        out[key].update(step_us=round(step * 1e3, 2), step_two_calls_us=round(two * 1e3, 2))
    del kc, vc, qs, kvr
    # head-start step: 200 sequences x 7 tokens, packed, no prefix
    B2, L2 = 200, 7
    T2 = B2 * L2
    set2 = T2 * (H + 2 * HK) * D * 2
    n2 = max(2, (300 << 20) // set2 + 1)
    qkv = torch.randn(n2, T2, (H + 2 * HK) * D, generator=gq, device=dev).to(torch.bfloat16)
    cu2 = torch.arange(0, T2 + 1, L2, dtype=torch.int32, device=dev)
    o2 = torch.empty(T2, H, D, dtype=torch.bfloat16, device=dev)

    def run_head():
        for i in range(n2):
            q, k, v = qkv[i].split([H * D, HK * D, HK * D], dim=-1)
            varlen_attention(q.view(T2, H, D), k.view(T2, HK, D), v.view(T2, HK, D), cu_seqlens_q=cu2,
                             cu_seqlens_k=cu2, max_seqlen_q=L2, softmax_scale=SCALE, causal=True, out=o2)

    ms2 = _graph_ms(run_head, 20) / n2
    out["headstart_200x7"] = dict(launch_us=round(ms2 * 1e3, 2), reference_published={"fa2_a10_us": 113})
    # the same step with its KV store (one 256-token block per sequence), bf16 and int8 output: the store riding in
    # the attention launch (prefill_attention_store; the W8A8 layer's store_kvcache + short_causal_attention pair,
    # kernels/fused_layer.py:643-667) against the two calls
    from voxcpm2_arabic_dialects_turbo_amd.ops import prefill_attention_store, store_kvcache

    kc2 = torch.zeros(B2, BS, HK, D, dtype=torch.bfloat16, device=dev)
    vc2 = torch.zeros_like(kc2)
    slots2 = (torch.arange(B2, device=dev).repeat_interleave(L2) * BS
              + torch.arange(L2, device=dev).repeat(B2)).to(torch.int32)
    inv2 = torch.rand(H * D, generator=gq, device=dev) + 0.5

    def run_head_step(quant, mode):  # mode: "riding", "two_calls" or "attention" (no store)
        def fn():
            for i in range(n2):
                q, k, v = qkv[i].split([H * D, HK * D, HK * D], dim=-1)
                q, k, v = q.view(T2, H, D), k.view(T2, HK, D), v.view(T2, HK, D)
                kw = dict(cu_seqlens_q=cu2, cu_seqlens_k=cu2, max_seqlen_q=L2, softmax_scale=SCALE, causal=True)
                if quant:
                    kw.update(quant=True, inv_smooth=inv2)
                if mode == "riding":
                    prefill_attention_store(q, k, v, kc2, vc2, slots2, **kw)
                else:
                    if mode == "two_calls":
                        store_kvcache(k, v, kc2, vc2, slots2)
                    varlen_attention(q, k, v, **kw)
        return fn

    for quant, key in ((False, "headstart_200x7"), (True, "headstart_200x7_int8")):
        if quant:
            out[key] = dict(launch_us=round(_graph_ms(run_head_step(True, "attention"), 20) / n2 * 1e3, 2))
        step = _graph_ms(run_head_step(quant, "riding"), 20) / n2
        two = _graph_ms(run_head_step(quant, "two_calls"), 20) / n2
        out[key].update(step_us=round(step * 1e3, 2), step_two_calls_us=round(two * 1e3, 2))
    del qkv, kc2, vc2
    # non-causal short rows (kernels/short_attn.py:1-10, 70-90): LocDiT 11 tokens and LocEnc 5 tokens per stream,
    # one stream per sequence of the 150-sequence decode batch; bf16 and the fused int8 output
    from voxcpm2_arabic_dialects_turbo_amd.kernels.short_attn import short_attention

    for name, L in (("locdit_150x11", 11), ("locenc_150x5", 5)):
        Bs = 150
        per = Bs * L * (H + 2 * HK) * D * 2
        ns = max(2, (300 << 20) // per + 1)
        qkv = torch.randn(ns, Bs, L, H + 2 * HK, D, generator=gq, device=dev).to(torch.bfloat16)
        for quant in (False, True):
            def run_short():
                for i in range(ns):
                    q, k, v = qkv[i].split([H, HK, HK], dim=2)
                    short_attention(q, k, v, SCALE, quant=quant)

            ms3 = _graph_ms(run_short, 20) / ns
            out[name + ("_int8" if quant else "")] = dict(launch_us=round(ms3 * 1e3, 2))
        del qkv
    return out


def bench_kv_copy(dev):
    """copy_kv_block_prefix over the model's cache layout (36 causal layers x K/V, 256-slot blocks): the voice-cloning
    prefix copy (44 entries x 50 tokens) and full-block copies (64 entries x 256 tokens); GB/s of bytes read and
    written."""
    import torch

    from voxcpm2_arabic_dialects_turbo_amd import _lib

    lib = _lib.load()
    blocks = 160
    kv = torch.empty(36, 2, blocks, BS, HK, D, dtype=torch.bfloat16, device=dev)
    kv.view(-1)[:] = 1
    out = {}
    perm = torch.randperm(blocks, generator=torch.Generator().manual_seed(53)).tolist()
    for name, n_entries, n_tok in (("prefix_44x50", 44, 50), ("full_64x256", 64, 256)):
        # the entries table is uploaded once (the wrapper's per-call pinned upload is not graph-capturable)
        pairs = torch.tensor([(perm[2 * i], perm[2 * i + 1], n_tok) for i in range(n_entries)], dtype=torch.int32,
                             device=dev)

        def run(pairs=pairs, n_entries=n_entries, n_tok=n_tok):
            _lib.check(lib.vox_copy_kv_block_prefix(kv.data_ptr(), 72, blocks, BS, HK * D, 2, pairs.data_ptr(),
                                                    n_entries, n_tok, _lib.stream_handle(dev)), "copy")

        ms = _graph_ms(run, 20)
        nbytes = 2 * n_entries * 72 * n_tok * HK * D * 2
        out[name] = dict(launch_us=round(ms * 1e3, 2), bytes=nbytes, gbs=round(nbytes / (ms * 1e-3) / 1e9, 1))
    return out


def bench_host_staging(dev, n_req: int = 200, reps: int = 200):
    """Host-side context staging (runner.py) for a burst of 200 cloned requests, the case the reference times at
    ~0.4 ms (nanovllm_voxcpm/engine/model_runner.py:851-854, its numpy staging with LoRA contexts, host time):
    each request a 50-token cached voice prompt plus 46 new tokens in one 256-token block, so the step's context
    has cu_seqlens, slots and block tables. Host microseconds per prepare_prefill_context call (numpy arrays written
    into the persistent page-locked staging buffer, one H2D copy queued, context set), and the same for the decode
    step's prepare_decode_context over the same 200 requests; a persistent StepStaging as the engine keeps."""
    import time

    import torch

    from voxcpm2_arabic_dialects_turbo_amd import runner
    from voxcpm2_arabic_dialects_turbo_amd.context import reset_context

    perm = torch.randperm(4 * n_req, generator=torch.Generator().manual_seed(57)).tolist()
    prefill = [runner.RunnerTask([perm[i]], 96, 50, BS) for i in range(n_req)]
    decode = [runner.RunnerTask([perm[i]], 97, 96, BS) for i in range(n_req)]
    staging = runner.StepStaging(dev)
    out = {}
    for name, fn, seqs in (("prefill_200_cloned", runner.prepare_prefill_context, prefill),
                           ("decode_200", runner.prepare_decode_context, decode)):
        for _ in range(20):
            fn(seqs, BS, device=dev, staging=staging)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn(seqs, BS, device=dev, staging=staging)
        host_us = (time.perf_counter() - t0) / reps * 1e6
        torch.cuda.synchronize()
        out[name] = dict(host_us=round(host_us, 1))
    reset_context()
    out["reference_published_ms"] = {"prefill_200_cloned": 0.4}
    return out


def cpu_config1(budget_s: float = 3.0):
    """Benchmark config 1 on the host cores: the oracle's decode (the reference tests' fp32 _attend over the gathered
    pages) for 1 sequence of context 512, 16 / 2 heads, fp32 caches of 4 blocks x 256 tokens in a random block order,
    N(0, 1) inputs from seed 1; repeated for ~budget_s seconds. Bytes: the same algorithmic units as the decode
    (fp32 elements)."""
    import torch

    from oracle import attention as ref

    gen = torch.Generator().manual_seed(1)
    table = torch.randperm(4, generator=gen).tolist()
    kc = torch.randn(4, BS, HK, D, generator=gen)
    vc = torch.randn(4, BS, HK, D, generator=gen)
    q = torch.randn(1, H, D, generator=gen)
    n, spent = 0, 0.0
    while spent < budget_s:
        t0 = time.perf_counter()
        ref.decode(q, kc, vc, [512], [table], SCALE)
        spent += time.perf_counter() - t0
        n += 1
    per = spent / n
    nbytes = 512 * HK * D * 4 * 2 + H * D * 4 * 2 + 4 * (1 + 2)
    return dict(us_per_call=round(per * 1e6, 1), gbs=round(nbytes / per / 1e9, 3), calls=n,
                sample="BASELINE config 1: oracle decode, 1 seq x ctx 512, fp32, torch on CPU")


def _cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(w, budget_s: float):
    """The oracle's torch path (fp32, as the reference's tests compute it) on the host cores over a bounded sample of
    the same decode step: layer after layer (store + decode of 150 sequences) until the budget is spent; plus
    benchmark config 1 (the reference's CPU-runnable case)."""
    import torch

    from oracle import attention as ref

    # every core this process may run on (os.cpu_count() counts the whole host, which a container's CPU share can
    # be far below; both are recorded)
    cpu_count = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else cpu_count
    torch.set_num_threads(usable)
    threads = torch.get_num_threads()
    lens = w.lens
    tables = [t.block_table + [-1] * (8 - len(t.block_table)) for t in w.tasks]
    slots = torch.tensor([ref.slot_of(t.block_table, t.seq_length - 1, BS) for t in w.tasks])
    done, spent = 0, 0.0
    while done < w.LAYERS and spent < budget_s:
        kc, vc = w.layers[done].k_cache.cpu(), w.layers[done].v_cache.cpu()
        q, k, v = (x.cpu() for x in w.views(done))
        t0 = time.perf_counter()
        ref.store_kvcache(k, v, kc, vc, slots)
        ref.decode(q.float(), kc, vc, lens, tables, SCALE)
        spent += time.perf_counter() - t0
        done += 1
    nbytes = done * (decode_bytes(lens) + store_bytes(len(lens)))
    return dict(value=round(nbytes / spent / 1e9, 3), unit="GB/s", cores=threads, kind="port",
                cpu_count=cpu_count, affinity_cpus=usable, threads=threads, cpu_model=_cpu_model(),
                sample=f"{done} of 28 layers of the config-4 decode step (store + decode, 150 sequences), "
                       f"torch fp32 on CPU, {spent:.1f} s",
                ms_per_step_extrapolated=round(spent / done * 28 * 1e3, 1),
                config1=cpu_config1())


TRAFFIC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "decode_config4_hbm_traffic.md")


def _profiled_traffic():
    """HBM bytes of one decode call, as measured by the rocprofv3 FETCH_SIZE / WRITE_SIZE runs summarized in
    profiles/ (copy-calibrated; the line `traffic_bytes_per_call: N`); None when no summary is present."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            m = re.search(r"traffic_bytes_per_call:\s*(\d+)", f.read())
    except OSError:
        return None
    return int(m.group(1)) if m else None


def _progress(msg: str) -> None:
    """A progress line on stderr (stdout carries only the result line)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs on a single MI355X and has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    from voxcpm2_arabic_dialects_turbo_amd import _lib

    _lib.load()
    if args.calibrate_copy:
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    res = bench_decode(args, dev)
    value = res["step_bytes"] / (res["ms_per_step"] * 1e-3) / 1e9
    achieved = res["launch_bytes"] / (res["launch_ms"] * 1e-3) / 1e9
    line = {
        "metric": "decode-attn HBM GB/s (%peak) @150 seqs; prefill attn TFLOP/s (%MFMA peak)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "BASELINE config 4: paged decode, 150 seqs x 28 layers, ctx U[256,2048], 16 q / 2 kv heads, "
                        "head_dim 128, bf16, 256-token blocks, 2048-block pool per layer; step = 28 "
                        "Attention.forward decode calls (store + decode) replayed as one HIP graph",
            "global_batch": DecodeWorkload.B,
            "seq_len": "U[256,2048]",
            "parallelism": "single GPU",
            "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
            "step_bytes": res["step_bytes"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_kernel<2, true> + decode_merge_kernel (one decode call)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": _profiled_traffic(),
            "launch_us": round(res["launch_ms"] * 1e3, 2),
            "launch_bytes": res["launch_bytes"],
        },
    }
    _progress(f"config 4 decode: {res['ms_per_step']:.4f} ms per step, {res['launch_ms'] * 1e3:.2f} us per call")
    if not args.decode_only:
        line["config3"] = bench_config3(dev)
        _progress(f"config 3: {line['config3']['launch_us']} us")
        line["config5"] = bench_config5(dev)
        _progress(f"config 5: {line['config5']['launch_us']} us")
        line["ceiling"] = bench_ceiling(dev, res["workload"])
        line["roofline"]["frac_of_decode_pattern_read"] = round(
            achieved / line["ceiling"]["decode_pattern_read_best_gbs"], 4)
        _progress(f"ceiling: {line['ceiling']}")
        line["prefill"] = bench_prefill(dev)
        _progress("prefill legs done")
        line["prefill"]["reference_shapes"] = bench_reference_shapes(dev)
        line["kv_block_prefix_copy"] = bench_kv_copy(dev)
        line["host_staging"] = bench_host_staging(dev)
        _progress("reference shapes, kv copy and host staging done")
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(res["workload"], args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
