"""Writes tests/golden/golden.npz: expected attention outputs on the reference tests' own shapes.

The reference repository commits no fixtures for this path and its attention functions cannot run here (they need
flash-attn and a CUDA GPU), so the expected outputs are computed in float64 by a per-(query, head) numpy loop that
shares no code with oracle/attention.py: scores = K_g q_h * scale, masked, exp(s - max) / sum. The inputs are not
stored; they are regenerated from the seeds below by ``inputs(case)`` (torch CPU generator, N(0, 1), rounded to
bf16 except the fp32 decode case), and a SHA-256 of the regenerated inputs is stored so a changed generator is
caught instead of silently compared.

Cases (shapes from the reference tests, tests/test_kernel_references.py):
- ``paged_prefill`` (:179-207): lens (new, total) = (5, 5), (7, 300), (1, 261); tables [[6, 0], [3, 5], [1, 7]];
  8 pages of 256; causal, bottom-right aligned; all 16 heads stored.
- ``short_causal`` (:210-228): packed lens [1, 7, 16, 32, 3], causal over own tokens; heads 0, 7, 8, 15 stored.
- ``dense`` (:229-237): B = 6, L = 5, non-causal; heads 0, 7, 8, 15 stored.
- ``decode_c1`` (benchmark config 1): 1 sequence, context 512, 4 blocks in random order, fp32.

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import os

import numpy as np
import torch

H, HK, D, PAGE = 16, 2, 128, 256
G = H // HK
SCALE = D ** -0.5
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "golden.npz")
STORED_HEADS = [0, 7, 8, 15]


def _randn(gen, *shape, dtype=torch.bfloat16):
    return torch.randn(*shape, generator=gen, dtype=torch.float32).to(dtype)


def inputs(case: str) -> dict:
    """The seeded inputs of ``case`` (CPU tensors)."""
    if case == "paged_prefill":
        gen = torch.Generator().manual_seed(1001)
        lens = [(5, 5), (7, 300), (1, 261)]
        T = sum(n for n, _ in lens)
        return dict(q=_randn(gen, T, H, D), k_cache=_randn(gen, 8, PAGE, HK, D), v_cache=_randn(gen, 8, PAGE, HK, D),
                    tables=torch.tensor([[6, 0], [3, 5], [1, 7]], dtype=torch.int32),
                    cu_q=torch.tensor([0, 5, 12, 13], dtype=torch.int32),
                    cu_k=torch.tensor([0, 5, 305, 566], dtype=torch.int32), max_q=7)
    if case == "short_causal":
        gen = torch.Generator().manual_seed(1002)
        lens = [1, 7, 16, 32, 3]
        T = sum(lens)
        cu = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32)
        return dict(q=_randn(gen, T, H, D), k=_randn(gen, T, HK, D), v=_randn(gen, T, HK, D), cu=cu, max_q=32)
    if case == "dense":
        gen = torch.Generator().manual_seed(1003)
        B, L = 6, 5
        return dict(q=_randn(gen, B, L, H, D), k=_randn(gen, B, L, HK, D), v=_randn(gen, B, L, HK, D))
    if case == "decode_c1":
        gen = torch.Generator().manual_seed(1)
        return dict(q=_randn(gen, 1, H, D, dtype=torch.float32),
                    k_cache=_randn(gen, 4, PAGE, HK, D, dtype=torch.float32),
                    v_cache=_randn(gen, 4, PAGE, HK, D, dtype=torch.float32),
                    tables=torch.randperm(4, generator=gen).to(torch.int32).view(1, 4),
                    lens=torch.tensor([512], dtype=torch.int32))
    raise KeyError(case)


def digest(inp: dict) -> str:
    h = hashlib.sha256()
    for key in sorted(inp):
        v = inp[key]
        if isinstance(v, torch.Tensor):
            h.update(key.encode())
            h.update(v.contiguous().view(torch.uint8).numpy().tobytes() if v.dtype == torch.bfloat16
                     else v.contiguous().numpy().tobytes())
    return h.hexdigest()


def _one_row(qv: np.ndarray, K: np.ndarray, V: np.ndarray, visible: int) -> np.ndarray:
    """float64 attention of one query vector over the first `visible` keys of K / V ([n, D])."""
    s = (K[:visible] @ qv) * SCALE
    e = np.exp(s - s.max())
    return (e @ V[:visible]) / e.sum()


def _seq(q: np.ndarray, K: np.ndarray, V: np.ndarray, causal: bool) -> np.ndarray:
    nq, nk = q.shape[0], K.shape[0]
    out = np.zeros((nq, H, D))
    for i in range(nq):
        visible = nk - nq + i + 1 if causal else nk
        for h in range(H):
            out[i, h] = _one_row(q[i, h], K[:, h // G], V[:, h // G], visible)
    return out


def _pages(cache: np.ndarray, table, n: int) -> np.ndarray:
    rows = [cache[int(table[j // PAGE]), j % PAGE] for j in range(n)]
    return np.stack(rows)


def expected(case: str, inp: dict) -> np.ndarray:
    f64 = {k: (v.double().numpy() if isinstance(v, torch.Tensor) and v.is_floating_point() else v)
           for k, v in inp.items()}
    if case == "paged_prefill":
        outs = []
        cu_q, cu_k = inp["cu_q"].tolist(), inp["cu_k"].tolist()
        for b in range(3):
            nk = cu_k[b + 1] - cu_k[b]
            K = _pages(f64["k_cache"], inp["tables"][b].tolist(), nk)
            V = _pages(f64["v_cache"], inp["tables"][b].tolist(), nk)
            outs.append(_seq(f64["q"][cu_q[b]:cu_q[b + 1]], K, V, causal=True))
        return np.concatenate(outs)
    if case == "short_causal":
        cu = inp["cu"].tolist()
        return np.concatenate([_seq(f64["q"][a:b], f64["k"][a:b], f64["v"][a:b], causal=True)
                               for a, b in zip(cu[:-1], cu[1:])])[:, STORED_HEADS]
    if case == "dense":
        return np.stack([_seq(f64["q"][b], f64["k"][b], f64["v"][b], causal=False)
                         for b in range(f64["q"].shape[0])])[:, :, STORED_HEADS]
    if case == "decode_c1":
        n = int(inp["lens"][0])
        K = _pages(f64["k_cache"], inp["tables"][0].tolist(), n)
        V = _pages(f64["v_cache"], inp["tables"][0].tolist(), n)
        return _seq(f64["q"], K, V, causal=True)
    raise KeyError(case)


CASES = ("paged_prefill", "short_causal", "dense", "decode_c1")


def main() -> None:
    arrays = {}
    for case in CASES:
        inp = inputs(case)
        arrays[f"{case}__out"] = expected(case, inp).astype(np.float32)
        arrays[f"{case}__sha256"] = np.array(digest(inp))
    np.savez_compressed(OUT, **arrays)
    print(OUT, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main()
