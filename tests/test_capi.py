"""The C ABI on the CPU: libvoxattn.so loads, exports every function include/vox_attn.h declares with the ABI
version the bindings expect, and rejects bad arguments with VOX_EINVAL before touching the GPU (no launches)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from voxcpm2_arabic_dialects_turbo_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "vox_attn.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vox_[a-z0-9_]+)\s*\(", text)))


def test_header_and_bindings_agree():
    assert _declared() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert lib.vox_abi_version() == _lib.ABI_VERSION


def test_only_one_hip_runtime_is_mapped():
    """The library binds to the HIP runtime torch loaded (same SONAME), never a second copy."""
    _lib.load()
    maps = open("/proc/self/maps").read()
    paths = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(paths) <= 1, paths


def _err():
    return _lib.load().vox_last_error().decode()


def test_store_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    assert lib.vox_store_kvcache(None, None, 256, 256, None, None, 10, None, 0, 2, 128, None) == _lib.VOX_OK  # empty
    assert lib.vox_store_kvcache(None, None, 256, 256, None, None, 10, None, 4, 2, 128, None) == _lib.VOX_EINVAL
    assert "null pointer" in _err()
    p = ctypes.c_void_p(16)  # never dereferenced: the checks fail first
    assert lib.vox_store_kvcache(p, p, 100, 256, p, p, 10, p, 4, 2, 128, None) == _lib.VOX_EINVAL
    assert "row stride" in _err()
    assert lib.vox_store_kvcache(p, p, 256, 256, p, p, 0, p, 4, 2, 128, None) == _lib.VOX_EINVAL


def _decode(**over):
    p = ctypes.c_void_p(256)
    a = dict(q=p, qs=16 * 128, kc=p, vc=p, nb=4, bs=256, bt=p, bts=8, mb=8, lens=p, b=2, h=16, hk=2, d=128,
             scale=0.088, plan=0, ws=p, wsb=1 << 30, out=p, stream=None)
    a.update(over)
    return _lib.load().vox_decode_attn(*a.values())


def test_decode_rejects_unsupported_shapes():
    assert _decode(b=0) == _lib.VOX_OK
    for over, msg in [(dict(d=64), "head_dim"), (dict(hk=4, h=16), "num_kv_heads"), (dict(h=32), "num_heads"),
                      (dict(bs=100), "block_size"), (dict(bts=4), "block table"),
                      (dict(wsb=10), "workspace"), (dict(qs=100), "row stride"), (dict(lens=None), "null"),
                      (dict(scale=float("nan")), "finite"), (dict(plan=3), "plan mode"),
                      (dict(plan=-1), "plan mode")]:
        assert _decode(**over) == _lib.VOX_EINVAL, over
        assert msg in _err(), (over, _err())


def _decode_store(**over):
    p = ctypes.c_void_p(256)
    a = dict(q=p, qs=16 * 128, key=p, value=p, ks=20 * 128, vs=20 * 128, slots=p, kc=p, vc=p, nb=4, bs=256, bt=p, bts=8,
             mb=8, lens=p, b=2, h=16, hk=2, d=128, scale=0.088, plan=0, ws=p, wsb=1 << 30, out=p, stream=None)
    a.update(over)
    return _lib.load().vox_decode_attn_store(*a.values())


def test_decode_store_rejects_bad_arguments():
    """The decode call with the store folded in: the store's own checks (rows 16-byte aligned, strides in whole
    16-byte pieces and at least one row) before the decode's, and an empty batch is a no-op."""
    assert _decode_store(b=0) == _lib.VOX_OK
    for over, msg in [(dict(key=None), "null"), (dict(slots=None), "null"), (dict(ks=100), "key / value"),
                      (dict(vs=128), "key / value"), (dict(value=ctypes.c_void_p(264)), "key / value"),
                      (dict(d=64), "head_dim"), (dict(wsb=10), "workspace"), (dict(lens=None), "null"),
                      (dict(plan=7), "plan mode")]:
        assert _decode_store(**over) == _lib.VOX_EINVAL, over
        assert msg in _err(), (over, _err())


def test_decode_workspace_and_grid_choice():
    lib = _lib.load()
    assert lib.vox_decode_workspace_bytes(0) == 0
    grid = lib.vox_decode_workgroups()
    assert grid > 0  # one workgroup per CU: 256 on an MI355X, also the fallback without a GPU
    def need(b, g):
        up = lambda x: -(-x // 256) * 256
        s = min(b, 512)  # sequences per launch
        # fp32 partials (one per sequence and workgroup), the step layout, plan records (4 KiB per workgroup)
        return up((s + g) * (16 * 128 + 32) * 4) + up((s + 2) * 4) + up(g * 1024 * 4)
    for b in (1, 40, 150, 512, 5000):
        assert lib.vox_decode_workspace_bytes(b) == need(b, grid)
    lib.vox_set_decode_workgroups(7)
    try:
        assert lib.vox_decode_workgroups() == 7
        assert lib.vox_decode_workspace_bytes(150) == need(150, 7)
    finally:
        lib.vox_set_decode_workgroups(0)
    assert lib.vox_decode_workgroups() == grid


def test_prefill_rejects_bad_arguments():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    # valid apart from the fake pointers: never passed unmodified (it would launch)
    args = [p, 2048, p, p, 256, 256, None, None, 0, 0, None, 0, 0, p, p, 2, 16, 0, 0, 16, 2, 128, 0.088, 1, p, 2048,
            0, None, 0, None]
    bad = list(args)
    bad[21] = 64  # head_dim
    assert lib.vox_prefill_attn(*bad) == _lib.VOX_EINVAL and "head_dim" in _err()
    bad = list(args)
    bad[13] = None  # only one cu_seqlens
    assert lib.vox_prefill_attn(*bad) == _lib.VOX_EINVAL and "cu_seqlens" in _err()
    bad = list(args)
    bad[19], bad[20] = 16, 3
    assert lib.vox_prefill_attn(*bad) == _lib.VOX_EINVAL and "multiple" in _err()
    bad = list(args)
    bad[2] = None  # packed mode without key
    assert lib.vox_prefill_attn(*bad) == _lib.VOX_EINVAL and "key/value" in _err()
    paged = list(args)  # paged varlen with a workspace below vox_prefill_workspace_bytes: rejected, no launch
    paged[2:4] = [None, None]
    paged[6:13] = [p, p, 64, 256, p, 8, 8]
    paged[27:29] = [p, 16]
    assert lib.vox_prefill_attn(*paged) == _lib.VOX_EINVAL and "workspace" in _err()
    paged[27:29] = [p, 1 << 30]
    paged[26] = 5  # not a plan mode
    assert lib.vox_prefill_attn(*paged) == _lib.VOX_EINVAL and "plan mode" in _err()
    assert lib.vox_prefill_workspace_bytes(2) == lib.vox_decode_workspace_bytes(2) > 16
    zero = list(args)
    zero[15] = 0  # empty batch: nothing to do
    assert lib.vox_prefill_attn(*zero) == _lib.VOX_OK


def test_prefill_store_rejects_bad_arguments_before_launching():
    """The packed prefill with the store riding in it checks every argument of both parts before it launches
    anything; nothing to attend and nothing to store is a no-op."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    # q, q stride, key, value, key/value strides, slots, k/v cache, num_slots, num_tokens, cu_q, cu_k, batch,
    # max_seqlen_q, H, HK, D, scale, causal, out, out stride, stream (fake pointers: never passed unmodified)
    args = [p, 2560, p, p, 2560, 2560, p, p, p, 1 << 17, 100, p, p, 2, 64, 16, 2, 128, 0.088, 1, p, 2048, None]
    for i, val, msg in [(17, 64, "head_dim"), (2, None, "null"), (6, None, "null"), (11, None, "null"),
                        (4, 200, "row strides"), (9, 0, "empty cache"), (13, -1, "negative"), (10, -5, "negative"),
                        (20, None, "null out"), (21, 100, "out row stride"), (16, 3, "multiple")]:
        bad = list(args)
        bad[i] = val
        assert lib.vox_prefill_attn_store(*bad) == _lib.VOX_EINVAL, (i, val)
        assert msg in _err(), (i, val, _err())
    empty = list(args)
    empty[13], empty[10] = 0, 0  # no sequences, no rows
    assert lib.vox_prefill_attn_store(*empty) == _lib.VOX_OK


def test_prefill_int8_rejects_bad_arguments():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    # valid apart from the fake pointers: never passed unmodified (it would launch)
    args = [p, 2048, p, p, 256, 256, None, None, 0, 0, None, 0, 0, p, p, 2, 16, 0, 0, 16, 2, 128, 0.088, 1, None, p,
            2048, p, 32, None, 0, None]
    bad = list(args)
    bad[20], bad[19] = 4, 16  # four KV heads: one workgroup would need 1024 threads
    assert lib.vox_prefill_attn_int8(*bad) == _lib.VOX_EINVAL and "num_kv_heads" in _err()
    bad = list(args)
    bad[27] = None  # no scale output
    assert lib.vox_prefill_attn_int8(*bad) == _lib.VOX_EINVAL and "out_scale" in _err()
    bad = list(args)
    bad[26] = 2046  # row stride not a multiple of 4
    assert lib.vox_prefill_attn_int8(*bad) == _lib.VOX_EINVAL and "out_q" in _err()
    bad = list(args)
    bad[24] = ctypes.c_void_p(260)  # inv_smooth not 16-byte aligned
    assert lib.vox_prefill_attn_int8(*bad) == _lib.VOX_EINVAL and "inv_smooth" in _err()
    bad = list(args)
    bad[21] = 64  # head_dim, from the shared prefill checks
    assert lib.vox_prefill_attn_int8(*bad) == _lib.VOX_EINVAL and "head_dim" in _err()
    bad = list(args)
    bad[28] = -1  # negative num_tokens
    assert lib.vox_prefill_attn_int8(*bad) == _lib.VOX_EINVAL and "num_tokens" in _err()
    bad = list(args)
    bad[13], bad[14], bad[17], bad[18], bad[28] = None, None, 16, 16, 31  # uniform lengths: T must be batch x 16
    assert lib.vox_prefill_attn_int8(*bad) == _lib.VOX_EINVAL and "num_tokens" in _err()
    long_ = list(args)  # a shape the two-pass form serves (8 causal sequences of up to 412 tokens)
    long_[15], long_[16], long_[28] = 8, 412, 2033
    need = lib.vox_prefill_int8_workspace_bytes(2033, 8, 412, 16, 2, 128, 1)
    assert need == 2033 * 16 * 128 * 2
    bad = list(long_)
    bad[29], bad[30] = p, need - 16  # workspace given but too small: rejected before any launch
    assert lib.vox_prefill_attn_int8(*bad) == _lib.VOX_EINVAL and "workspace" in _err()
    bad[29], bad[30] = ctypes.c_void_p(264), need  # not 16-byte aligned
    assert lib.vox_prefill_attn_int8(*bad) == _lib.VOX_EINVAL and "workspace" in _err()
    zero = list(args)
    zero[15] = 0
    assert lib.vox_prefill_attn_int8(*zero) == _lib.VOX_OK


def test_prefill_int8_two_pass_choice():
    """The int8 output runs as two passes (bf16 attention, then a quantization pass) only for causal calls whose
    16-row items outnumber the CUs over sequences of 16+ items (the fallback CU count without a GPU is 256); short
    steps, non-causal rows and rows of more than 2048 values keep the fused epilogue (0 bytes)."""
    lib = _lib.load()
    ws = lib.vox_prefill_int8_workspace_bytes
    assert ws(2033, 8, 412, 16, 2, 128, 1) == 2033 * 16 * 128 * 2  # config 2: 52 tiles x 8 sequences
    assert ws(2033, 8, 412, 16, 2, 128, 0) == 0                     # non-causal
    assert ws(2024, 44, 46, 16, 2, 128, 1) == 0                     # 44 x 46: 6 tiles per sequence
    assert ws(750, 150, 5, 16, 2, 128, 1) == 0                      # LocEnc-sized steps
    assert ws(600, 2, 300, 16, 2, 128, 1) == 0                      # 76 items: fewer than the CUs
    assert ws(2033, 8, 412, 32, 2, 128, 1) == 0                     # 4096 values per token row
    assert ws(0, 8, 412, 16, 2, 128, 1) == 0


@pytest.mark.skipif(__import__("torch").cuda.is_available(), reason="launches with placeholder pointers: CPU only")
@pytest.mark.parametrize("int8", [False, True])
def test_prefill_with_one_kv_head_for_128_query_heads_returns_a_status(int8):
    """A group of 128 query heads per KV head is accepted by the argument checks; the launcher must pick a
    workgroup shape without dividing by zero (64 / group) and come back with a status: VOX_EHIP here, where the
    launch itself fails for want of a GPU. Run in a child process, so a crash fails the test instead of pytest."""
    import subprocess
    import sys

    fn = "vox_prefill_attn_int8" if int8 else "vox_prefill_attn"
    tail = "None, p, 128 * 128, p, 4, None, 0, None" if int8 else "p, 128 * 128, 0, None, 0, None"
    code = f"""
import ctypes, sys
sys.path.insert(0, {os.path.dirname(os.path.dirname(os.path.abspath(__file__)))!r})
from voxcpm2_arabic_dialects_turbo_amd import _lib
lib = _lib.load()
p = ctypes.c_void_p(256)
st = lib.{fn}(p, 128 * 128, p, p, 128, 128, None, None, 0, 0, None, 0, 0, p, p, 2, 16, 0, 0, 128, 1, 128, 0.088, 1,
              {tail})
print(st)
"""
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stderr[-2000:])
    assert int(r.stdout.split()[-1]) in (_lib.VOX_OK, _lib.VOX_EHIP)


def test_copy_kv_block_prefix_rejects_bad_arguments():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    args = [p, 72, 64, 256, 256, 2, p, 3, 256, None]  # valid apart from the fake pointers: never passed unmodified
    bad = list(args)
    bad[5] = 4  # 4-byte elements
    assert lib.vox_copy_kv_block_prefix(*bad) == _lib.VOX_EINVAL and "2 only" in _err()
    bad = list(args)
    bad[0] = None
    assert lib.vox_copy_kv_block_prefix(*bad) == _lib.VOX_EINVAL and "null" in _err()
    bad = list(args)
    bad[1] = 70000
    assert lib.vox_copy_kv_block_prefix(*bad) == _lib.VOX_EINVAL and "planes" in _err()
    bad = list(args)
    bad[3] = 0
    assert lib.vox_copy_kv_block_prefix(*bad) == _lib.VOX_EINVAL and "shape" in _err()
    for i, v in ((7, 0), (8, 0), (1, 0)):  # nothing to copy: no launch
        ok = list(args)
        ok[i] = v
        assert lib.vox_copy_kv_block_prefix(*ok) == _lib.VOX_OK


def test_flash_attn_entry_points_take_flash_attn_2_8_3_positional_order():
    """flash-attn 2.8.3's parameter order (the version the reference pins), so positional callers bind the same
    arguments; options this path does not implement raise instead of being ignored. The checks run before any device
    work, so CPU tensors show which check fired."""
    import inspect

    import torch

    from voxcpm2_arabic_dialects_turbo_amd import ops

    def names(fn):
        return list(inspect.signature(fn).parameters)

    assert names(ops.flash_attn_func) == ["q", "k", "v", "dropout_p", "softmax_scale", "causal", "window_size",
                                          "softcap", "alibi_slopes", "deterministic", "return_attn_probs"]
    assert names(ops.flash_attn_varlen_func) == [
        "q", "k", "v", "cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q", "max_seqlen_k", "dropout_p", "softmax_scale",
        "causal", "window_size", "softcap", "alibi_slopes", "deterministic", "return_attn_probs", "block_table"]
    assert names(ops.flash_attn_with_kvcache) == [
        "q", "k_cache", "v_cache", "k", "v", "rotary_cos", "rotary_sin", "cache_seqlens", "cache_batch_idx",
        "cache_leftpad", "block_table", "softmax_scale", "causal", "window_size", "softcap", "rotary_interleaved",
        "alibi_slopes", "num_splits", "return_softmax_lse"]
    q = torch.zeros(1, 3, 16, 128, dtype=torch.bfloat16)
    kv = torch.zeros(1, 3, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="dropout_p"):
        ops.flash_attn_func(q, kv, kv, 0.1)  # 4th positional is dropout_p, as in flash-attn
    with pytest.raises(NotImplementedError, match="window_size"):
        ops.flash_attn_func(q, kv, kv, window_size=(4, 0))
    with pytest.raises(ValueError, match="GPU"):  # dropout_p = 0.0 passes the option check; then: no GPU here
        ops.flash_attn_func(q, kv, kv, 0.0, None, False)
    cu = torch.tensor([0, 3], dtype=torch.int32)
    with pytest.raises(NotImplementedError, match="dropout_p"):
        ops.flash_attn_varlen_func(q[0], kv[0], kv[0], cu, cu, 3, 3, 0.5)
    cache = torch.zeros(2, 256, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="k="):
        ops.flash_attn_with_kvcache(q, cache, cache, kv, kv)


def test_python_errors_carry_the_library_message():
    with pytest.raises(ValueError, match="head_dim"):
        _lib.check(_decode(d=64), "decode_attn")


def test_prefill_store_paged_rejects_bad_arguments_before_launching():
    """The paged prefill with the store riding in it (a mixed step's call) checks every argument of both parts,
    the workspace and the plan mode included, before it launches anything; nothing to attend and nothing to store is
    a no-op."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    # q, q stride, key, value, key/value strides, slots, num_tokens, k/v cache, num_blocks, block_size, table, table
    # stride, max_blocks, cu_q, cu_k, batch, max_seqlen_q, H, HK, D, scale, causal, out, out stride, plan, workspace,
    # its bytes, stream (fake pointers: never passed unmodified)
    args = [p, 2560, p, p, 2560, 2560, p, 100, p, p, 512, 256, p, 8, 8, p, p, 2, 64, 16, 2, 128, 0.088, 1, p, 2048, 0,
            p, 1 << 30, None]
    for i, val, msg in [(21, 64, "head_dim"), (2, None, "null"), (6, None, "null"), (12, None, "null"),
                        (15, None, "null"), (4, 200, "row strides"), (10, 0, "empty cache"), (17, -1, "negative"),
                        (7, -5, "negative"), (24, None, "null out"), (25, 100, "out row stride"), (20, 3, "multiple"),
                        (13, 4, "block table"), (26, 5, "plan mode"), (28, 16, "workspace")]:
        bad = list(args)
        bad[i] = val
        assert lib.vox_prefill_attn_store_paged(*bad) == _lib.VOX_EINVAL, (i, val)
        assert msg in _err(), (i, val, _err())
    empty = list(args)
    empty[17], empty[7] = 0, 0  # no sequences, no rows
    assert lib.vox_prefill_attn_store_paged(*empty) == _lib.VOX_OK
