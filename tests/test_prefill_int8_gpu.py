"""GPU parity of the prefill kernel's int8 output epilogue (the quant=True modes of the reference's Triton
paged_prefill_attention, short_causal_attention and short_attention) against the oracle: fp32 attention, then the
reference's per-token quantization (oracle.attention.quantize_rows).

Bounds per token row (scale = the oracle's per-token scale):
- scale: relative error <= 1e-2 (the amax of an output whose elements are within the attention tolerance);
- dequantized int8 vs the fp32 oracle output: <= 0.51 * scale + 0.02 * max|ref| everywhere (the reference test's own
  bound, tests/test_kernel_references.py:206-209), and mean error <= 0.3 * mean(scale) + 2e-3;
- int8 codes: at most 1% of them differ from the oracle's codes by more than one step.
"""

from __future__ import annotations

import pytest
import torch

from oracle import attention as ref
from tests._util import D, H, HK, paged_pool, randn, uniform_lens
from tests.golden import make_golden
from voxcpm2_arabic_dialects_turbo_amd import _lib
from voxcpm2_arabic_dialects_turbo_amd.kernels.prefill_attn import paged_prefill_attention
from voxcpm2_arabic_dialects_turbo_amd.kernels.short_attn import short_attention, short_causal_attention
from voxcpm2_arabic_dialects_turbo_amd.ops import varlen_attention

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = D ** -0.5


def _check(out, want, what, inv_smooth=None):
    """out = (int8 [T, H*D], fp32 [T]) from the GPU; want = fp32 attention output [T, H*D] (or [T, H, D])."""
    q, scale = out
    T = scale.numel()
    assert q.dtype == torch.int8 and scale.dtype == torch.float32 and q.shape == (T, want.numel() // T)
    want = want.reshape(T, -1).float()
    q_ref, s_ref = ref.quantize_rows(want, inv_smooth)
    y = want if inv_smooth is None else want * inv_smooth.float().cpu()
    q, scale = q.cpu(), scale.cpu()
    rel = ((scale - s_ref).abs() / s_ref).max().item()
    assert rel <= 1e-2, f"{what}: scale relative error {rel:.3g}"
    err = (ref.dequantize_rows(q, scale) - y).abs()
    bound = 0.51 * s_ref[:, None] + 0.02 * y.abs().max()
    assert bool((err <= bound).all()), f"{what}: dequantized error {err.max().item():.3g}"
    assert err.mean().item() <= 0.3 * s_ref.mean().item() + 2e-3, f"{what}: mean error {err.mean().item():.3g}"
    off = ((q.int() - q_ref.int()).abs() > 1).float().mean().item()
    assert off <= 0.01, f"{what}: {off:.2%} of codes more than one step from the oracle's"


@pytest.mark.parametrize("smooth", [False, True])
def test_paged_prefill_int8_reference_case(smooth):
    """tests/test_kernel_references.py:179-207 with quant=True (and an inv_smooth vector)."""
    inp = make_golden.inputs("paged_prefill")
    d = {k: (v.to(DEV) if isinstance(v, torch.Tensor) else v) for k, v in inp.items()}
    inv = (torch.rand(H * D, generator=torch.Generator().manual_seed(70)) + 0.5) if smooth else None
    out = paged_prefill_attention(d["q"], d["k_cache"], d["v_cache"], d["tables"], d["cu_q"], d["cu_k"], 7, SCALE,
                                  quant=True, inv_smooth=None if inv is None else inv.to(DEV))
    want = ref.varlen(inp["q"].float(), inp["cu_q"], inp["cu_k"], k_cache=inp["k_cache"], v_cache=inp["v_cache"],
                      block_tables=inp["tables"])
    _check(out, want, "paged prefill int8", inv)


def test_short_causal_int8_reference_case():
    """tests/test_kernel_references.py:210-228 with quant=True: packed lens [1, 7, 16, 32, 3]."""
    inp = make_golden.inputs("short_causal")
    out = short_causal_attention(inp["q"].to(DEV), inp["k"].to(DEV), inp["v"].to(DEV), inp["cu"].to(DEV), 32, SCALE,
                                 quant=True)
    _check(out, ref.varlen(inp["q"].float(), inp["cu"], inp["cu"], k=inp["k"], v=inp["v"]), "short causal int8")


@pytest.mark.parametrize("L", [1, 5, 11, 16])
def test_short_non_causal_int8(L):
    """tests/test_kernel_references.py:230-236 with quant=True: 6 rows of L tokens, non-causal."""
    gen = torch.Generator().manual_seed(71 + L)
    q, k, v = randn(gen, 6, L, H, D), randn(gen, 6, L, HK, D), randn(gen, 6, L, HK, D)
    out = short_attention(q.to(DEV), k.to(DEV), v.to(DEV), SCALE, quant=True)
    _check(out, ref.dense(q.float(), k.float(), v.float()).reshape(6 * L, -1), f"short L={L} int8")


def test_config2_packed_int8_with_smoothing():
    """benchmark config 2 shape (8 packed causal sequences, L ~ U[64, 512]), int8 output with inv_smooth."""
    gen = torch.Generator().manual_seed(72)
    lens = uniform_lens(gen, 8, 64, 512)
    T = sum(lens)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    q, k, v = randn(gen, T, H, D), randn(gen, T, HK, D), randn(gen, T, HK, D)
    inv = torch.rand(H * D, generator=gen) * 2 + 0.25
    out = varlen_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV),
                           max_seqlen_q=max(lens), softmax_scale=SCALE, causal=True, quant=True,
                           inv_smooth=inv.to(DEV))
    _check(out, ref.varlen(q.float(), cu, cu, k=k, v=v), "config 2 int8", inv)


def test_paged_int8_one_kv_head_and_zero_length_rows():
    """8 query heads over 1 KV head (tensor parallel 2), paged with a cached prefix, and padded zero-length
    sequences, whose rows are not written."""
    gen = torch.Generator().manual_seed(73)
    nq, nk = [9, 0, 40, 0, 1], [300, 0, 40, 0, 77]
    kc, vc, tables = paged_pool(gen, [max(n, 1) for n in nk], 12, hk=1)
    T = sum(nq)
    q = randn(gen, T, 8, D)
    cu_q = torch.tensor([0] + torch.tensor(nq).cumsum(0).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + torch.tensor(nk).cumsum(0).tolist(), dtype=torch.int32)
    out = paged_prefill_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), tables.to(DEV), cu_q.to(DEV), cu_k.to(DEV),
                                  max(nq), SCALE, quant=True)
    want = ref.varlen(q.float(), cu_q, cu_k, k_cache=kc, v_cache=vc, block_tables=tables)
    _check(out, want, "HK=1 paged int8")


def test_int8_codes_round_half_to_even_at_exact_ties():
    """One key per sequence and a zero query make p = exp2(0) = 1 and o = v exactly; with one element 127 per token
    the scale is exactly 1, so the codes are rint(v) for values placed on half-integers (2.5 -> 2, -3.5 -> -4,
    0.5 -> 0, ...): round half to even, the oracle's torch.round, bit-exact."""
    gen = torch.Generator().manual_seed(74)
    B = 12
    ties = torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -3.5, 10.5, -10.5, 126.5, -126.5])
    v = ties[torch.randint(0, ties.numel(), (B, HK, D), generator=gen)]
    v[:, 0, 0] = 127.0  # the token's max |o| over all heads: scale = 127 / 127 = 1
    q, k = torch.zeros(B, H, D, dtype=torch.bfloat16), randn(gen, B, HK, D)
    cu = torch.arange(B + 1, dtype=torch.int32)
    out_q, scale = varlen_attention(q.to(DEV), k.to(DEV), v.to(torch.bfloat16).to(DEV), cu_seqlens_q=cu.to(DEV),
                                    cu_seqlens_k=cu.to(DEV), max_seqlen_q=1, softmax_scale=SCALE, causal=True,
                                    quant=True)
    want = v.repeat_interleave(H // HK, dim=1).reshape(B, H * D)  # o of head h is v of its kv head
    q_ref, s_ref = ref.quantize_rows(want.float())
    assert torch.equal(scale.cpu(), s_ref) and float(s_ref[0]) == 1.0
    assert torch.equal(out_q.cpu(), q_ref), "codes differ from round-half-to-even"
    flat_v, flat_q = want.flatten(), out_q.cpu().flatten()
    for val, code in ((2.5, 2), (-3.5, -4), (0.5, 0), (-1.5, -2), (126.5, 126)):
        hit = flat_v == val
        assert bool(hit.any()) and bool((flat_q[hit] == code).all()), f"{val} -> {code}"


def test_int8_large_ragged_grid_in_per_xcd_order():
    """int8 output on a grid of 128 q tiles x 8 sequences (>= 1024 workgroups: per-XCD work order) with ragged
    lengths."""
    gen = torch.Generator().manual_seed(75)
    lens = [2048, 33, 1200, 700, 5, 1999, 64, 1500]
    T = sum(lens)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    q, k, v = randn(gen, T, H, D), randn(gen, T, HK, D), randn(gen, T, HK, D)
    out = varlen_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV),
                           max_seqlen_q=max(lens), softmax_scale=SCALE, causal=True, quant=True)
    _check(out, ref.varlen(q.float(), cu, cu, k=k, v=v), "per-XCD order int8")


@pytest.mark.parametrize("bs", [None, 256, 96])
def test_int8_sixteen_row_halves_over_several_key_tiles(bs):
    """Grids small enough for one workgroup per CU take 16-row waves (8 tokens per workgroup at 8 heads per KV
    head): 3 causal sequences of 150-333 tokens over several key tiles, packed keys and paged caches (block size
    256: one block id per key tile; 96: per-piece block ids), with an inv_smooth vector."""
    gen = torch.Generator().manual_seed(76 + (bs or 0))
    lens = [333, 150, 271]
    T = sum(lens)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    q = randn(gen, T, H, D)
    inv = torch.rand(H * D, generator=gen) + 0.5
    if bs is None:
        k, v = randn(gen, T, HK, D), randn(gen, T, HK, D)
        out = varlen_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV),
                               max_seqlen_q=max(lens), softmax_scale=SCALE, causal=True, quant=True,
                               inv_smooth=inv.to(DEV))
        want = ref.varlen(q.float(), cu, cu, k=k, v=v)
    else:
        kc, vc, tables = paged_pool(gen, lens, sum((n + bs - 1) // bs for n in lens) + 2, block_size=bs)
        out = paged_prefill_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), tables.to(DEV), cu.to(DEV), cu.to(DEV),
                                      max(lens), SCALE, quant=True, inv_smooth=inv.to(DEV))
        want = ref.varlen(q.float(), cu, cu, k_cache=kc, v_cache=vc, block_tables=tables)
    _check(out, want, f"16-row int8, block_size {bs}", inv)


@pytest.mark.parametrize("two_pass", [True, False])
@pytest.mark.parametrize("bs,h,hk", [(None, 16, 2), (256, 16, 2), (96, 16, 2), (None, 8, 1)])
def test_int8_rank_major_grid_beyond_one_item_per_cu(bs, h, hk, two_pass, monkeypatch):
    """Causal grids of 16-row halves with more items than CUs (256 on an MI355X) over sequences of 16+ items: by
    default two passes (the bf16 kernel into a scratch buffer, then the per-token quantization); with the library's
    workspace query forced to 0, the fused epilogue in the rank-major grid, the heaviest q tile of every sequence
    first. Packed keys and paged caches (block size 256 and 96), one and two KV heads, sequences of very different
    lengths (the short ones' high ranks are empty)."""
    lib = _lib.load()
    # 63 items per sequence x 6 sequences > 256 CUs: the two-pass form unless the query is forced to 0
    assert lib.vox_prefill_int8_workspace_bytes(sum([333, 150, 271, 500, 9, 310]), 6, 500, h, hk, D, 1) > 0
    if not two_pass:
        monkeypatch.setattr(lib, "vox_prefill_int8_workspace_bytes", lambda *a: 0)
    gen = torch.Generator().manual_seed(81 + (bs or 0) + hk)
    lens = [333, 150, 271, 500, 9, 310]
    assert 256 < -(-max(lens) // (64 // (h // hk))) * len(lens) <= 512
    T = sum(lens)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    q = randn(gen, T, h, D)
    inv = torch.rand(h * D, generator=gen) + 0.5
    if bs is None:
        k, v = randn(gen, T, hk, D), randn(gen, T, hk, D)
        out = varlen_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu_seqlens_q=cu.to(DEV), cu_seqlens_k=cu.to(DEV),
                               max_seqlen_q=max(lens), softmax_scale=SCALE, causal=True, quant=True,
                               inv_smooth=inv.to(DEV))
        want = ref.varlen(q.float(), cu, cu, k=k, v=v)
    else:
        kc, vc, tables = paged_pool(gen, lens, sum((n + bs - 1) // bs for n in lens) + 2, block_size=bs, hk=hk)
        out = paged_prefill_attention(q.to(DEV), kc.to(DEV), vc.to(DEV), tables.to(DEV), cu.to(DEV), cu.to(DEV),
                                      max(lens), SCALE, quant=True, inv_smooth=inv.to(DEV))
        want = ref.varlen(q.float(), cu, cu, k_cache=kc, v_cache=vc, block_tables=tables)
    _check(out, want, f"rank-major int8, block_size {bs}, {h}/{hk} heads, two passes {two_pass}", inv)


def test_int8_two_pass_codes_round_half_to_even_at_exact_ties():
    """The two-pass form (long causal sequences, more 16-row items than CUs) on exact ties: a zero query gives every
    visible key the same weight, and each sequence's values are the same at every key position, so o = v exactly
    (the fp32 sums of half-integers are exact, and o is representable in bf16); with one element 127 per token the
    scale is exactly 1 and the codes are rint(v), round half to even, bit-exact against the oracle."""
    lib = _lib.load()
    gen = torch.Generator().manual_seed(79)
    lens = [400, 390, 380, 370, 360, 350]
    T = sum(lens)
    assert lib.vox_prefill_int8_workspace_bytes(T, len(lens), max(lens), H, HK, D, 1) > 0  # the two-pass form
    ties = torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -3.5, 10.5, -10.5, 126.5, -126.5])
    t = ties[torch.randint(0, ties.numel(), (len(lens), HK, D), generator=gen)]
    t[:, 0, 0] = 127.0
    v = torch.cat([t[b].expand(n, HK, D) for b, n in enumerate(lens)])
    q, k = torch.zeros(T, H, D, dtype=torch.bfloat16), randn(gen, T, HK, D)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    out_q, scale = varlen_attention(q.to(DEV), k.to(DEV), v.to(torch.bfloat16).to(DEV), cu_seqlens_q=cu.to(DEV),
                                    cu_seqlens_k=cu.to(DEV), max_seqlen_q=max(lens), softmax_scale=SCALE,
                                    causal=True, quant=True)
    want = v.repeat_interleave(H // HK, dim=1).reshape(T, H * D)
    q_ref, s_ref = ref.quantize_rows(want.float())
    assert torch.equal(scale.cpu(), s_ref) and bool((s_ref == 1.0).all())
    assert torch.equal(out_q.cpu(), q_ref), "codes differ from round-half-to-even"


def test_int8_two_pass_with_uniform_lengths():
    """The two-pass form without cu_seqlens (batch x uniform lengths, the flash_attn_func layout): 6 causal
    sequences of 400 tokens, token count batch x 400, against the oracle with inv_smooth."""
    lib = _lib.load()
    B, L = 6, 400
    assert lib.vox_prefill_int8_workspace_bytes(B * L, B, L, H, HK, D, 1) > 0
    gen = torch.Generator().manual_seed(82)
    q, k, v = randn(gen, B * L, H, D), randn(gen, B * L, HK, D), randn(gen, B * L, HK, D)
    inv = torch.rand(H * D, generator=gen) + 0.5
    out = varlen_attention(q.to(DEV), k.to(DEV), v.to(DEV), cu_seqlens_q=None, cu_seqlens_k=None, max_seqlen_q=L,
                           batch=B, uniform_seqlen_q=L, uniform_seqlen_k=L, softmax_scale=SCALE, causal=True,
                           quant=True, inv_smooth=inv.to(DEV))
    cu = torch.arange(0, B * L + 1, L, dtype=torch.int32)
    _check(out, ref.varlen(q.float(), cu, cu, k=k, v=v), "uniform two-pass int8", inv)


def test_int8_two_pass_and_fused_forms_agree_on_one_shape(monkeypatch):
    """The two forms of the int8 output on the same inputs: the two-pass form quantizes the bf16-rounded o (as the
    reference's flash-attn + quantize path does), the fused epilogue the fp32 o (as the reference's Triton QUANT
    epilogue does, kernels/prefill_attn.py:84-92). Which one runs depends on the shape and the CU count, so they must
    agree: scales within bf16 rounding of the row maximum (relative 2^-8) and codes within one step."""
    lib = _lib.load()
    gen = torch.Generator().manual_seed(83)
    lens = [333, 150, 271, 500, 9, 310]
    T = sum(lens)
    assert lib.vox_prefill_int8_workspace_bytes(T, len(lens), max(lens), H, HK, D, 1) > 0
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=DEV)
    q, k, v = (randn(gen, T, n, D).to(DEV) for n in (H, HK, HK))
    inv = (torch.rand(H * D, generator=gen) + 0.5).to(DEV)

    def run():
        return varlen_attention(q, k, v, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens),
                                softmax_scale=SCALE, causal=True, quant=True, inv_smooth=inv)

    q2, s2 = run()
    monkeypatch.setattr(lib, "vox_prefill_int8_workspace_bytes", lambda *a: 0)
    q1, s1 = run()
    torch.cuda.synchronize()
    rel = ((s1 - s2).abs() / s1).max().item()
    assert rel <= 2.0 ** -8, f"scales of the two forms differ by {rel:.3g} (relative)"
    step = (q1.int() - q2.int()).abs().max().item()
    assert step <= 1, f"codes of the two forms differ by {step} steps"


@pytest.mark.parametrize("two_pass", [True, False])
def test_int8_output_rows_past_num_tokens_are_never_written(two_pass, monkeypatch):
    """A caller whose num_tokens is below cu_seqlens_q[batch] (the library cannot read device memory to check) gets
    the rows below num_tokens computed and nothing written past them: the guard bytes after out_q, out_scale and the
    two-pass scratch stay as they were."""
    lib = _lib.load()
    gen = torch.Generator().manual_seed(84)
    lens = [400, 390, 380, 370, 360, 350]
    T = sum(lens)
    cut = T - 500  # the caller's num_tokens: the last sequences' rows fall past it
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=DEV)
    q, k, v = (randn(gen, T, n, D).to(DEV) for n in (H, HK, HK))
    guard = 4096
    out_q = torch.full((cut * H * D + guard,), 77, dtype=torch.int8, device=DEV)
    out_s = torch.full((cut + guard,), 7.0, dtype=torch.float32, device=DEV)
    ws_bytes = lib.vox_prefill_int8_workspace_bytes(cut, len(lens), max(lens), H, HK, D, 1) if two_pass else 0
    assert (ws_bytes > 0) == two_pass
    ws = torch.full((ws_bytes + guard,), 0x5A, dtype=torch.uint8, device=DEV)
    st = lib.vox_prefill_attn_int8(q.data_ptr(), q.stride(0), k.data_ptr(), v.data_ptr(), k.stride(0), v.stride(0),
                                   None, None, 0, 0, None, 0, 0, cu.data_ptr(), cu.data_ptr(), len(lens), max(lens), 0,
                                   0, H, HK, D, SCALE, 1, None, out_q.data_ptr(), H * D, out_s.data_ptr(), cut,
                                   ws.data_ptr() if two_pass else None, ws_bytes, _lib.stream_handle(q.device))
    _lib.check(st, "prefill_attn_int8")
    torch.cuda.synchronize()
    assert bool((out_q[cut * H * D:] == 77).all()), "int8 rows written past num_tokens"
    assert bool((out_s[cut:] == 7.0).all()), "scales written past num_tokens"
    assert bool((ws[ws_bytes:] == 0x5A).all()), "two-pass scratch written past num_tokens rows"
    full_q, full_s = varlen_attention(q, k, v, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens),
                                      softmax_scale=SCALE, causal=True, quant=True)
    if not two_pass:  # (the full call takes the two-pass form for this shape)
        monkeypatch.setattr(lib, "vox_prefill_int8_workspace_bytes", lambda *a: 0)
        full_q, full_s = varlen_attention(q, k, v, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens),
                                          softmax_scale=SCALE, causal=True, quant=True)
    assert torch.equal(out_q[:cut * H * D].view(cut, H * D), full_q[:cut]) and torch.equal(out_s[:cut], full_s[:cut])


@pytest.mark.parametrize("h,hk,smooth", [(16, 2, False), (16, 2, True), (16, 1, True)])
def test_int8_two_pass_codes_equal_the_quantized_bf16_output(h, hk, smooth):
    """The two-pass form of the long causal shapes (the bf16 kernel into the workspace, then the per-token
    quantization) quantizes the bf16 output the plain call gives, bit for bit: codes and scales equal the oracle's
    quantization of that output (config-2-like lengths)."""
    gen = torch.Generator().manual_seed(85 + h + hk)
    lens = [412, 393, 361, 205, 108, 405, 75, 74]
    T = sum(lens)
    lib = _lib.load()
    assert lib.vox_prefill_int8_workspace_bytes(T, len(lens), max(lens), h, hk, D, 1) > 0
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=DEV)
    q, k, v = (randn(gen, T, n, D).to(DEV) for n in (h, hk, hk))
    inv = (torch.rand(h * D, generator=gen) + 0.5).to(DEV) if smooth else None
    kw = dict(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens), softmax_scale=SCALE, causal=True)
    codes, scales = varlen_attention(q, k, v, quant=True, inv_smooth=inv, **kw)
    o = varlen_attention(q, k, v, **kw)
    torch.cuda.synchronize()
    q_ref, s_ref = ref.quantize_rows(o.reshape(T, -1).float().cpu(), None if inv is None else inv.cpu())
    assert torch.equal(scales.cpu(), s_ref), "scales differ from the quantized bf16 output's"
    assert torch.equal(codes.cpu(), q_ref), "codes differ from the quantized bf16 output's"


@pytest.mark.parametrize("h,hk", [(4, 2), (8, 2), (2, 1), (32, 1), (64, 2), (64, 1), (128, 1)])
def test_int8_group_sizes(h, hk):
    """The int8 epilogue over group sizes 2, 4, 32, 64 and 128 (the model's 8 and 16 are covered above): one scale
    per token over all h heads, where a 16-row wave may hold part of one token's heads (groups above 16) and the
    token rows span both kv halves of the workgroup (hk = 2). Rows of more than 16 heads take the fused epilogue."""
    gen = torch.Generator().manual_seed(95 + h + hk)
    lens = [1, 70, 129, 33]
    T = sum(lens)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    q, k, v = (randn(gen, T, n, D) for n in (h, hk, hk))
    out = varlen_attention(q.to(DEV), k.to(DEV), v.to(DEV), quant=True, cu_seqlens_q=cu.to(DEV),
                           cu_seqlens_k=cu.to(DEV), max_seqlen_q=max(lens), softmax_scale=SCALE, causal=True)
    torch.cuda.synchronize()
    _check(out, ref.varlen(q.float(), cu, cu, k=k, v=v), f"int8 H={h} HK={hk}")


def test_int8_two_pass_in_a_hip_graph_replays_like_eager():
    """The two-pass int8 form captured in a HIP graph (its workspace allocated inside the capture) and replayed four
    times, with eager calls on other inputs between the replays: every replay equals the eager result bit for bit."""
    gen = torch.Generator().manual_seed(86)
    lens = [333, 150, 271, 500, 9, 310]
    T = sum(lens)
    assert _lib.load().vox_prefill_int8_workspace_bytes(T, len(lens), max(lens), H, HK, D, 1) > 0
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=DEV)
    q, k, v = (randn(gen, T, n, D).to(DEV) for n in (H, HK, HK))
    q2 = randn(gen, T, H, D).to(DEV)
    kw = dict(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens), softmax_scale=SCALE, causal=True, quant=True)
    eager = varlen_attention(q, k, v, **kw)
    eager2 = varlen_attention(q2, k, v, **kw)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static = varlen_attention(q, k, v, **kw)
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static[0], eager[0]) and torch.equal(static[1], eager[1]), f"replay {r}"
        other = varlen_attention(q2, k, v, **kw)
        torch.cuda.synchronize()
        assert torch.equal(other[0], eager2[0]) and torch.equal(other[1], eager2[1])


@pytest.mark.parametrize("case", ["headstart", "ranked", "two_pass", "one_kv_head", "padded_slots", "unaligned_caches"])
def test_int8_prefill_with_the_store_riding_in_it_equals_store_then_prefill(case, monkeypatch):
    """prefill_attention_store(quant=True) without a block table (the W8A8 layer's store_kvcache +
    short_causal_attention pair, nanovllm_voxcpm/kernels/fused_layer.py:643-667, as one call: the copy rides in the
    int8 launch) against store_kvcache then varlen_attention(quant=True): codes, scales and both caches bit-identical.
    Cases: the head-start step (200 sequences of 7 tokens, the fused epilogue's plain grid); 20 x 128 tokens with no
    two-pass workspace (the fused epilogue's rank-major grid); config-2-like lengths (the two-pass form: the copy in
    the bf16 pass); one kv head; padding and out-of-range slots; caches that are not 16-byte aligned (the two
    calls)."""
    from tests._util import BLOCK
    from voxcpm2_arabic_dialects_turbo_amd.ops import prefill_attention_store, store_kvcache

    gen = torch.Generator().manual_seed(99)
    hk = 1 if case == "one_kv_head" else HK
    lens = {"headstart": [7] * 200, "ranked": [128] * 20}.get(case, [412, 393, 361, 205, 108, 405, 75, 74])
    T = sum(lens)
    kc, vc, tables = paged_pool(gen, lens, sum(-(-n // BLOCK) for n in lens) + 2, hk=hk)
    qkv = randn(gen, T, (H + 2 * hk) * D).to(DEV)
    q, k, v = qkv.split([H * D, hk * D, hk * D], dim=-1)
    q, k, v = q.view(T, H, D), k.view(T, hk, D), v.view(T, hk, D)
    slots = torch.cat([torch.tensor([ref.slot_of(tables[b].tolist(), j, BLOCK) for j in range(n)])
                       for b, n in enumerate(lens)]).to(torch.int32)
    if case == "padded_slots":
        slots[::5] = -1
        slots[2::9] = kc.shape[0] * BLOCK + 3  # past the cache
    inv = (torch.rand(H * D, generator=gen) + 0.5).to(DEV)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32, device=DEV)
    kc1, vc1 = kc.to(DEV), vc.to(DEV)
    kc2, vc2 = kc1.clone(), vc1.clone()
    if case == "unaligned_caches":
        def shifted(c):
            buf = torch.empty(c.numel() + 4, dtype=c.dtype, device=DEV)
            view = buf[4:].view(c.shape)
            view.copy_(c)
            return view
        kc1, vc1 = shifted(kc1), shifted(vc1)
    kw = dict(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens), softmax_scale=SCALE, causal=True)
    if case == "ranked":  # the fused epilogue rather than the two passes this shape gets a workspace for
        lib = _lib.load()
        assert lib.vox_prefill_int8_workspace_bytes(T, len(lens), max(lens), H, hk, D, 1) > 0
        monkeypatch.setattr(lib, "vox_prefill_int8_workspace_bytes", lambda *a: 0)
    codes, scales = prefill_attention_store(q, k, v, kc1, vc1, slots.to(DEV), quant=True, inv_smooth=inv, **kw)
    store_kvcache(k, v, kc2, vc2, slots.to(DEV))
    codes2, scales2 = varlen_attention(q, k, v, quant=True, inv_smooth=inv, **kw)
    torch.cuda.synchronize()
    assert torch.equal(codes, codes2) and torch.equal(scales, scales2), f"{case}: int8 output differs"
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), f"{case}: caches differ from store_kvcache's"


@pytest.mark.parametrize("case", ["prefix50", "two_pass", "one_kv_head", "blocks_of_32"])
def test_paged_int8_prefill_with_the_store_riding_in_it_equals_store_then_prefill(case):
    """prefill_attention_store(quant=True) through block tables (the W8A8 layer's store_kvcache +
    paged_prefill_attention(quant=True) pair of its eager prefix-cache steps, nanovllm_voxcpm/kernels/fused_layer.py:
    619-641, as one call: the launch reads each sequence's new keys from the rows and copies them) against
    store_kvcache then varlen_attention(quant=True) over the caches: codes, scales and both caches bit-identical.
    Cases: 44 sequences of 46 new tokens over 50 cached ones (the reference's shape; the fused epilogue, its tile that
    straddles the first new key written to the cache by its readers); config-2-like lengths with no prefix (the
    two-pass form); one kv head over prefixes; 32-token blocks (the two calls)."""
    from voxcpm2_arabic_dialects_turbo_amd.ops import prefill_attention_store, store_kvcache

    gen = torch.Generator().manual_seed(101)
    hk = 1 if case == "one_kv_head" else HK
    bs = 32 if case == "blocks_of_32" else 256
    if case == "two_pass":
        nq, pre = [412, 393, 361, 205, 108, 405, 75, 74], [0] * 8
    elif case == "prefix50":
        nq, pre = [46] * 44, [50] * 44
    else:
        nq, pre = [30, 77, 5, 120], [0, 13, 64, 200]
    nk = [a + b for a, b in zip(nq, pre)]
    T = sum(nq)
    kc, vc, tables = paged_pool(gen, nk, sum(-(-n // bs) for n in nk) + 2, block_size=bs, hk=hk)
    qkv = randn(gen, T, (H + 2 * hk) * D).to(DEV)
    q, k, v = qkv.split([H * D, hk * D, hk * D], dim=-1)
    q, k, v = q.view(T, H, D), k.view(T, hk, D), v.view(T, hk, D)
    slots = torch.tensor([ref.slot_of(tables[b].tolist(), j, bs) for b in range(len(nk))
                          for j in range(nk[b] - nq[b], nk[b])], dtype=torch.int32).to(DEV)
    inv = (torch.rand(H * D, generator=gen) + 0.5).to(DEV)
    cu_q = torch.tensor([0] + torch.tensor(nq).cumsum(0).tolist(), dtype=torch.int32, device=DEV)
    cu_k = torch.tensor([0] + torch.tensor(nk).cumsum(0).tolist(), dtype=torch.int32, device=DEV)
    bt = tables.to(DEV)
    kc1, vc1 = kc.to(DEV), vc.to(DEV)
    kc2, vc2 = kc1.clone(), vc1.clone()
    kw = dict(cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=max(nq), softmax_scale=SCALE, causal=True,
              quant=True, inv_smooth=inv)
    codes, scales = prefill_attention_store(q, k, v, kc1, vc1, slots, block_table=bt, **kw)
    store_kvcache(k, v, kc2, vc2, slots)
    codes2, scales2 = varlen_attention(q, None, None, block_table=bt, k_cache=kc2, v_cache=vc2, **kw)
    torch.cuda.synchronize()
    assert torch.equal(codes, codes2) and torch.equal(scales, scales2), f"{case}: int8 output differs"
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), f"{case}: caches differ from store_kvcache's"
