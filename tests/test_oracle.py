"""Pins the CPU oracle (oracle/) before anything is checked against it: closed forms, brute force on tiny inputs, an
independent library routine (torch SDPA in float64), the reference tests' known-answer cases, the golden vectors,
and planted mistakes that these checks must catch. CPU only."""

from __future__ import annotations

import itertools
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as ref
from oracle import context as ctxref
from tests._util import randn
from tests.golden import make_golden

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden.npz")


# --- brute force and library cross-checks -------------------------------------------------------------------------

def _brute(q, k, v, causal, scale):
    """Pure-Python float64 attention, one (query, head) at a time; GQA by explicit index h // (H // HK)."""
    nq, H, D = q.shape
    nk, HK, _ = k.shape
    G = H // HK
    out = torch.zeros(nq, H, D, dtype=torch.float64)
    for i, h in itertools.product(range(nq), range(H)):
        g = h // G
        last = nk - nq + i if causal else nk - 1
        s = [scale * sum(float(q[i, h, d]) * float(k[j, g, d]) for d in range(D)) for j in range(last + 1)]
        mx = max(s)
        w = [math.exp(x - mx) for x in s]
        tot = sum(w)
        for d in range(D):
            out[i, h, d] = sum(w[j] * float(v[j, g, d]) for j in range(last + 1)) / tot
    return out.reshape(nq, -1)


@pytest.mark.parametrize("nq,nk,causal", [(1, 1, True), (3, 3, True), (2, 5, True), (4, 6, False), (1, 6, True)])
def test_attend_matches_brute_force(nq, nk, causal):
    gen = torch.Generator().manual_seed(nq * 10 + nk)
    q = torch.randn(nq, 4, 3, generator=gen, dtype=torch.float64)
    k = torch.randn(nk, 2, 3, generator=gen, dtype=torch.float64)
    v = torch.randn(nk, 2, 3, generator=gen, dtype=torch.float64)
    torch.testing.assert_close(ref.attend(q, k, v, causal, scale=0.7), _brute(q, k, v, causal, 0.7),
                               rtol=1e-12, atol=1e-12)


def _sdpa(q, k, v, causal, scale):
    """torch's SDPA (math, float64) with GQA expanded by index_select(h // G) and an explicit bottom-right mask."""
    nq, H, D = q.shape
    nk, HK, _ = k.shape
    idx = torch.arange(H) // (H // HK)
    ke, ve = k.index_select(1, idx), v.index_select(1, idx)
    mask = None
    if causal:
        mask = torch.arange(nk)[None, :] <= (nk - nq + torch.arange(nq))[:, None]
    o = F.scaled_dot_product_attention(q.transpose(0, 1), ke.transpose(0, 1), ve.transpose(0, 1), attn_mask=mask,
                                       scale=scale)
    return o.transpose(0, 1).reshape(nq, -1)


@pytest.mark.parametrize("nq,nk,causal", [(7, 300, True), (5, 5, True), (1, 261, True), (11, 11, False)])
def test_attend_matches_sdpa_float64(nq, nk, causal):
    gen = torch.Generator().manual_seed(nk)
    q = torch.randn(nq, 16, 128, generator=gen, dtype=torch.float64)
    k = torch.randn(nk, 2, 128, generator=gen, dtype=torch.float64)
    v = torch.randn(nk, 2, 128, generator=gen, dtype=torch.float64)
    torch.testing.assert_close(ref.attend(q, k, v, causal), _sdpa(q, k, v, causal, 128 ** -0.5),
                               rtol=1e-10, atol=1e-10)


# --- closed forms ----------------------------------------------------------------------------------------------------

def test_single_key_returns_its_value_per_group():
    q = torch.randn(3, 16, 128, dtype=torch.float64)
    k = torch.randn(1, 2, 128, dtype=torch.float64)
    v = torch.randn(1, 2, 128, dtype=torch.float64)
    o = ref.attend(q[:1], k, v, causal=True).view(1, 16, 128)
    for h in range(16):
        assert torch.equal(o[0, h], v[0, h // 8])


def test_identical_keys_average_the_values():
    v = torch.randn(9, 2, 128, dtype=torch.float64)
    k = torch.ones(9, 2, 128, dtype=torch.float64)
    q = torch.randn(9, 16, 128, dtype=torch.float64)
    o = ref.attend(q, k, v, causal=False).view(9, 16, 128)
    torch.testing.assert_close(o[4, 3], v[:, 0].mean(0))
    oc = ref.attend(q, k, v, causal=True).view(9, 16, 128)
    for i in range(9):  # causal, nq == nk: query i averages values 0..i
        torch.testing.assert_close(oc[i, 12], v[:i + 1, 1].mean(0))
    torch.testing.assert_close(oc[0, 0], v[0, 0])  # query 0 sees only key 0


def test_two_key_softmax_matches_the_logistic_weight():
    """Pins the scale: with two keys, o = sigmoid(scale * (s0 - s1)) v0 + (1 - ...) v1."""
    q = torch.zeros(1, 1, 128, dtype=torch.float64)
    q[0, 0, 0] = 3.0
    k = torch.zeros(2, 1, 128, dtype=torch.float64)
    k[0, 0, 0], k[1, 0, 0] = 1.0, -0.5
    v = torch.randn(2, 1, 128, dtype=torch.float64)
    w0 = 1.0 / (1.0 + math.exp(-(128 ** -0.5) * (3.0 * 1.0 - 3.0 * -0.5)))
    torch.testing.assert_close(ref.attend(q, k, v, causal=False).view(128), w0 * v[0, 0] + (1 - w0) * v[1, 0])


def test_gqa_head_h_reads_kv_head_h_div_group():
    k = torch.randn(5, 2, 128, dtype=torch.float64)
    v = torch.stack([torch.zeros(5, 128), torch.ones(5, 128)], 1).double()
    q = torch.randn(2, 16, 128, dtype=torch.float64)
    o = ref.attend(q, k, v, causal=True).view(2, 16, 128)
    assert torch.equal(o[:, :8], torch.zeros(2, 8, 128, dtype=torch.float64))
    torch.testing.assert_close(o[:, 8:], torch.ones(2, 8, 128, dtype=torch.float64))


def test_decode_equals_varlen_with_one_query():
    gen = torch.Generator().manual_seed(5)
    kc, vc = randn(gen, 6, 256, 2, 128, dtype=torch.float32), randn(gen, 6, 256, 2, 128, dtype=torch.float32)
    tables = torch.tensor([[4, 1, -1], [0, 5, 2]], dtype=torch.int32)
    lens = [300, 700]
    q = randn(gen, 2, 16, 128, dtype=torch.float32)
    dec = ref.decode(q, kc, vc, lens, tables)
    var = ref.varlen(q, [0, 1, 2], [0, 300, 1000], k_cache=kc, v_cache=vc, block_tables=tables)
    torch.testing.assert_close(dec, var)


def test_page_gather_is_the_slot_formula():
    gen = torch.Generator().manual_seed(6)
    cache = randn(gen, 5, 32, 2, 128, dtype=torch.float32)
    table = [3, 0, 4]
    got = ref.gather_pages(cache, table, 70)
    flat = cache.view(-1, 2, 128)
    for j in range(70):
        assert torch.equal(got[j], flat[ref.slot_of(table, j, 32)])


def test_store_known_answer_case_from_the_reference():
    """Slots of tests/test_kernel_references.py:240-257: each row lands at its slot, -1 skipped, nothing else."""
    gen = torch.Generator().manual_seed(3)
    k_cache = torch.zeros(4, 256, 2, 128, dtype=torch.bfloat16)
    v_cache = torch.zeros_like(k_cache)
    k, v = randn(gen, 9, 2, 128), randn(gen, 9, 2, 128)
    slots = [5, 300, 511, 512, 1023, -1, 0, 700, 256]
    ref.store_kvcache(k, v, k_cache, v_cache, torch.tensor(slots, dtype=torch.int32))
    fk, fv = k_cache.view(-1, 2, 128), v_cache.view(-1, 2, 128)
    for i, s in enumerate(slots):
        if s >= 0:
            assert torch.equal(fk[s], k[i]) and torch.equal(fv[s], v[i])
    assert int((fk.float().abs().sum((1, 2)) > 0).sum()) == 8


# --- golden vectors --------------------------------------------------------------------------------------------------

def _golden():
    return np.load(GOLDEN, allow_pickle=False)


@pytest.mark.parametrize("case", make_golden.CASES)
def test_golden_inputs_regenerate_identically(case):
    assert str(_golden()[f"{case}__sha256"]) == make_golden.digest(make_golden.inputs(case))


def test_oracle_reproduces_golden_vectors():
    g = _golden()
    inp = make_golden.inputs("paged_prefill")
    out = ref.varlen(inp["q"].float(), inp["cu_q"], inp["cu_k"], k_cache=inp["k_cache"], v_cache=inp["v_cache"],
                     block_tables=inp["tables"])
    np.testing.assert_allclose(out.numpy(), g["paged_prefill__out"], rtol=0, atol=2e-5)
    inp = make_golden.inputs("short_causal")
    out = ref.varlen(inp["q"].float(), inp["cu"], inp["cu"], k=inp["k"], v=inp["v"])
    np.testing.assert_allclose(out[:, make_golden.STORED_HEADS].numpy(), g["short_causal__out"], atol=2e-5)
    inp = make_golden.inputs("dense")
    out = ref.dense(inp["q"].float(), inp["k"].float(), inp["v"].float())
    np.testing.assert_allclose(out[:, :, make_golden.STORED_HEADS].numpy(), g["dense__out"], atol=2e-5)
    inp = make_golden.inputs("decode_c1")
    out = ref.decode(inp["q"], inp["k_cache"], inp["v_cache"], inp["lens"], inp["tables"])
    np.testing.assert_allclose(out.numpy(), g["decode_c1__out"], atol=2e-5)


# --- planted mistakes: each must fail at least one of the checks above --------------------------------------------

def _attend_gqa_modulo(q, k, v, causal, scale=None):  # wrong: head h reads kv head h % HK
    return _with_kv_index(q, k, v, causal, scale, torch.arange(q.shape[1]) % k.shape[1])


def _with_kv_index(q, k, v, causal, scale, idx):
    H = q.shape[1]
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    att = torch.einsum("qhd,khd->hqk", q, k.index_select(1, idx)) * scale
    if causal:
        n_q, n_k = q.shape[0], k.shape[0]
        mask = torch.arange(n_k)[None, :] > (n_k - n_q + torch.arange(n_q))[:, None]
        att = att.masked_fill(mask[None], float("-inf"))
    return torch.einsum("hqk,khd->qhd", att.softmax(-1), v.index_select(1, idx)).reshape(q.shape[0], -1)


def _attend_top_left(q, k, v, causal, scale=None):  # wrong: causal mask aligned top-left
    H, HK = q.shape[1], k.shape[1]
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    k, v = k.repeat_interleave(H // HK, 1), v.repeat_interleave(H // HK, 1)
    att = torch.einsum("qhd,khd->hqk", q, k) * scale
    if causal:
        mask = torch.arange(k.shape[0])[None, :] > torch.arange(q.shape[0])[:, None]
        att = att.masked_fill(mask[None], float("-inf"))
    return torch.einsum("hqk,khd->qhd", att.softmax(-1), v).reshape(q.shape[0], -1)


def _attend_no_scale(q, k, v, causal, scale=None):  # wrong: scale dropped
    return ref.attend(q, k, v, causal, scale=1.0)


@pytest.mark.parametrize("wrong", [_attend_gqa_modulo, _attend_top_left, _attend_no_scale])
def test_planted_mistakes_are_caught(wrong):
    gen = torch.Generator().manual_seed(9)
    q = torch.randn(3, 16, 128, generator=gen, dtype=torch.float64)
    k = torch.randn(7, 2, 128, generator=gen, dtype=torch.float64)
    v = torch.randn(7, 2, 128, generator=gen, dtype=torch.float64)
    caught = not torch.allclose(wrong(q, k, v, True), _sdpa(q, k, v, True, 128 ** -0.5), atol=1e-6)
    g = _golden()
    inp = make_golden.inputs("paged_prefill")
    outs = []
    for b in range(3):
        cq, ck = inp["cu_q"].tolist(), inp["cu_k"].tolist()
        kb = ref.gather_pages(inp["k_cache"], inp["tables"][b], ck[b + 1] - ck[b]).float()
        vb = ref.gather_pages(inp["v_cache"], inp["tables"][b], ck[b + 1] - ck[b]).float()
        outs.append(wrong(inp["q"][cq[b]:cq[b + 1]].float(), kb, vb, True))
    caught_golden = not np.allclose(torch.cat(outs).view(13, 16, 128).numpy(), g["paged_prefill__out"], atol=1e-3)
    assert caught and caught_golden


# --- context definitions ------------------------------------------------------------------------------------------

class _Task:
    def __init__(self, table, length, cached):
        self.block_table, self.seq_length, self.num_cached_tokens = table, length, cached


def test_prefill_context_hand_computed():
    """block_size 4: a 6-token sequence with 3 cached tokens in blocks [7, 2], and a fresh 2-token one in [5]."""
    seqs = [_Task([7, 2], 6, 3), _Task([5], 2, 0)]
    pos, cu_q, cu_k, mq, mk, slots, tables = ctxref.prefill_context(4, seqs)
    assert pos == [3, 4, 5, 0, 1]
    assert (cu_q, cu_k, mq, mk) == ([0, 3, 5], [0, 6, 8], 3, 6)
    assert slots == [7 * 4 + 3, 2 * 4 + 0, 2 * 4 + 1, 5 * 4 + 0, 5 * 4 + 1]
    assert tables == [[7, 2], [5, -1]]  # a cached prefix: tables staged
    assert ctxref.prefill_context(4, [_Task([5], 2, 0)])[6] is None  # no prefix, no graphs: no tables
    assert ctxref.prefill_context(4, [_Task([], 3, 0)])[5] == []  # warm-up task: no slots


def test_decode_context_hand_computed():
    seqs = [_Task([7, 2], 6, 5), _Task([5], 4, 3), _Task([1, 3, 9], 9, 8)]
    pos, slots, lens, tables = ctxref.decode_context(4, seqs)
    assert pos == [5, 3, 8]
    assert slots == [2 * 4 + 1, 5 * 4 + 3, 9 * 4 + 0]
    assert lens == [6, 4, 9]
    assert tables == [[7, 2, -1], [5, -1, -1], [1, 3, 9]]


# --- int8 output epilogue (quantize_rows) -------------------------------------------------------------------------

def test_quantize_rows_closed_form_and_half_to_even():
    """amax 127 gives scale 1 exactly, so q = rint(y): halves go to the even neighbour (a round-half-away oracle
    would give -3, 3 for -2.5, 2.5)."""
    x = torch.tensor([[127.0, -2.5, 2.5, 3.5, -3.5, 0.49, 1.5, -126.5]])
    q, scale = ref.quantize_rows(x)
    assert scale.tolist() == [1.0]
    assert q.tolist() == [[127, -2, 2, 4, -4, 0, 2, -126]]
    assert q.dtype == torch.int8 and scale.dtype == torch.float32


def test_quantize_rows_zero_row_and_smoothing():
    q, scale = ref.quantize_rows(torch.zeros(1, 6))
    assert q.abs().sum() == 0 and scale.item() == pytest.approx(1e-6 / 127, rel=1e-6)
    inv = torch.tensor([1.0, 2.0, 0.5, 4.0])
    q, scale = ref.quantize_rows(torch.ones(2, 4), inv)  # y = inv_smooth itself: amax 4
    assert scale.tolist() == [float(np.float32(4.0) / np.float32(127.0))] * 2
    assert q[0].tolist() == [round(127 / 4), round(127 / 2), round(127 / 8), 127]


def test_quantize_rows_matches_an_elementwise_loop():
    """Per-element restatement in numpy float32 with Python's round (half to even) on random rows."""
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(5, 48, generator=gen) * torch.tensor([0.01, 1.0, 30.0, 1e-7, 5.0])[:, None]
    inv = torch.rand(48, generator=gen) + 0.5
    q, scale = ref.quantize_rows(x, inv)
    xs, invs = x.numpy().astype(np.float32), inv.numpy().astype(np.float32)
    for i in range(5):
        y = [np.float32(xs[i, j]) * invs[j] for j in range(48)]
        amax = max(max(abs(v) for v in y), np.float32(1e-6))
        s = np.float32(amax) / np.float32(127.0)
        assert np.float32(scale[i].item()) == s
        assert q[i].tolist() == [int(round(float(np.float32(v) / s))) for v in y]
        # the reference test's bound on the dequantized row (tests/test_kernel_references.py:206-209)
        err = (ref.dequantize_rows(q[i:i + 1], scale[i:i + 1]) - x[i:i + 1] * inv).abs()
        assert bool((err <= 0.51 * scale[i]).all())


# --- KV block-prefix copy --------------------------------------------------------------------------------------------

def test_kv_block_prefix_copy_known_answer():
    """Every element holds its own flat index, so each copied run is identified exactly: block dst's first n slots of
    every (layer, K/V) plane equal block src's, everything else is untouched; n is clipped to the block size and
    n <= 0 does nothing (reference: kernels/kv_copy.py:31-35)."""
    from oracle import kvcopy

    kv = torch.arange(3 * 2 * 5 * 4 * 2 * 3, dtype=torch.float64).reshape(3, 2, 5, 4, 2, 3)
    orig = kv.clone()
    kvcopy.copy_kv_block_prefix(kv, [(1, 3, 2), (0, 4, 9), (2, 2, 0), (3, 0, -1)])
    want = orig.clone()
    want[:, :, 3, :2] = orig[:, :, 1, :2]
    want[:, :, 4, :4] = orig[:, :, 0, :4]  # 9 clipped to the block size
    assert torch.equal(kv, want)
    # the flat formula of the reference's kernel: plane p, element o of the run -> p*plane + block*bstride + o
    flat, oflat = kv.reshape(6, -1), orig.reshape(6, -1)
    bstride = 4 * 2 * 3
    for p in range(6):
        for o in range(2 * 2 * 3):
            assert flat[p, 3 * bstride + o] == oflat[p, 1 * bstride + o]
