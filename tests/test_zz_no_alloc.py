"""The allocation-free decode entry point (vox_decode_attn_noalloc) against the workspace entry point
(vox_decode_attn): same kernels, so the outputs must agree bit for bit, on two calls in a row (the second with a
smaller batch, so the shared static scratch holds the first call's values), and within tolerance of the oracle."""

from __future__ import annotations

import pytest
import torch

from oracle import attention as ref
from tests._util import D, H, HK, attn_close, paged_pool, randn, uniform_lens
from voxcpm2_arabic_dialects_turbo_amd import _lib
from voxcpm2_arabic_dialects_turbo_amd.ops import decode_attention

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE = D ** -0.5


def _noalloc(q, kc, vc, lens, tables):
    lib = _lib.load()
    out = torch.empty(q.shape[0], H, D, dtype=torch.bfloat16, device=DEV)
    nb, bs = kc.shape[0], kc.shape[1]
    st = lib.vox_decode_attn_noalloc(q.data_ptr(), q.stride(0), kc.data_ptr(), vc.data_ptr(), nb, bs,
                                     tables.data_ptr(), tables.stride(0), tables.shape[1], lens.data_ptr(),
                                     q.shape[0], H, HK, D, SCALE, out.data_ptr(), _lib.stream_handle(out.device))
    _lib.check(st, "decode_attn_noalloc")
    return out


def test_noalloc_decode_matches_the_workspace_entry_point_on_two_calls():
    for seed, batch, lo, hi in ((140, 150, 256, 2048), (141, 37, 1, 700)):
        gen = torch.Generator().manual_seed(seed)
        lens = uniform_lens(gen, batch, lo, hi)
        kc, vc, tables = paged_pool(gen, lens, sum((n + 255) // 256 for n in lens) + 8)
        q = randn(gen, batch, H, D)
        q_d, kc_d, vc_d, t_d = q.to(DEV), kc.to(DEV), vc.to(DEV), tables.to(DEV)
        lens_d = torch.tensor(lens, dtype=torch.int32, device=DEV)
        got = _noalloc(q_d, kc_d, vc_d, lens_d, t_d)
        want = decode_attention(q_d, kc_d, vc_d, lens_d, t_d, SCALE)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"batch {batch}: allocation-free call differs from vox_decode_attn"
        attn_close(got, ref.decode(q.float(), kc, vc, lens, tables, SCALE), f"noalloc batch {batch}")


def test_noalloc_decode_rejects_a_scratch_need_beyond_the_static_array():
    lib = _lib.load()
    lib.vox_set_decode_workgroups(5000)  # partials for 512 + 5000 workgroups: beyond 16 MiB
    try:
        p = torch.empty(16, dtype=torch.uint8, device=DEV)
        st = lib.vox_decode_attn_noalloc(p.data_ptr(), 2048, p.data_ptr(), p.data_ptr(), 4, 256, p.data_ptr(), 8, 8,
                                         p.data_ptr(), 512, H, HK, D, SCALE, p.data_ptr(), None)
        assert st == _lib.VOX_EINVAL and "scratch" in lib.vox_last_error().decode()
    finally:
        lib.vox_set_decode_workgroups(0)


_CAPTURE_SCRIPT = r"""
import sys
sys.path.insert(0, {root!r})
import torch
from tests._util import D, H, HK, paged_pool, randn, uniform_lens
from voxcpm2_arabic_dialects_turbo_amd import _lib
from voxcpm2_arabic_dialects_turbo_amd.ops import decode_attention

dev = torch.device("cuda")
lib = _lib.load()
gen = torch.Generator().manual_seed(142)
B = 60
lens = uniform_lens(gen, B, 1, 1500)
kc, vc, tables = paged_pool(gen, lens, sum((n + 255) // 256 for n in lens) + 8)
kc, vc, tables = kc.to(dev), vc.to(dev), tables.to(dev)
lens_d = torch.tensor(lens, dtype=torch.int32, device=dev)
q = torch.zeros(B, H, D, dtype=torch.bfloat16, device=dev)
out = torch.empty(B, H, D, dtype=torch.bfloat16, device=dev)
s = torch.cuda.Stream()

def call():
    st = lib.vox_decode_attn_noalloc(q.data_ptr(), q.stride(0), kc.data_ptr(), vc.data_ptr(), kc.shape[0], 256,
                                     tables.data_ptr(), tables.stride(0), tables.shape[1], lens_d.data_ptr(), B, H,
                                     HK, D, D ** -0.5, out.data_ptr(), _lib.stream_handle(dev))
    assert st == 0, lib.vox_last_error()

torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    before = torch.cuda.memory_allocated()
    call()  # the process's first call: the scratch symbol is looked up inside the capture
    assert torch.cuda.memory_allocated() == before, "the allocation-free call allocated"
torch.cuda.synchronize()
for rep in range(3):
    q.copy_(randn(gen, B, H, D).to(dev))
    g.replay()
    torch.cuda.synchronize()
    got = out.clone()
    want = decode_attention(q, kc, vc, lens_d, tables, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(got, want), f"replay {{rep}} differs from the workspace entry point"
    before = torch.cuda.memory_allocated()
    call()
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before and torch.equal(out, want)
print("ok")
"""


def test_noalloc_first_call_inside_a_graph_capture_in_a_fresh_process():
    """The first allocation-free call of a process made inside a HIP graph capture (the scratch's device address is
    looked up there), the graph replayed over new queries with eager work between replays, each replay bit-identical
    to vox_decode_attn; torch's allocator sees no allocation from the entry point. A child process, so the lookup
    really is the process's first."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT.format(root=root)], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), (r.returncode, r.stdout[-1000:], r.stderr[-3000:])
