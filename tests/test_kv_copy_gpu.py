"""GPU parity of the KV block-prefix copy (HIP kernel 4) against the oracle: bit-exact."""

from __future__ import annotations

import pytest
import torch

from oracle import kvcopy
from voxcpm2_arabic_dialects_turbo_amd import _lib
from voxcpm2_arabic_dialects_turbo_amd.kernels.kv_copy import copy_kv_block_prefix

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _kv(shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)


def test_copy_model_shape_many_entries():
    """36 causal layers x K/V over 24 blocks of 256 slots (the model's cache layout): partial, full, clipped,
    dropped and single-token entries."""
    kv = _kv((36, 2, 24, 256, 2, 128), 80)
    entries = [(3, 10, 50), (5, 7, 256), (0, 23, 300), (1, 2, 0), (11, 12, 1), (13, 14, 129), (20, 21, -3)]
    kv_d = kv.to(DEV)
    copy_kv_block_prefix(kv_d, entries)
    kvcopy.copy_kv_block_prefix(kv, entries)
    assert torch.equal(kv_d.cpu(), kv)


def test_copy_two_byte_path_and_out_of_range_blocks():
    """Slots of 4 elements (not a 16-byte multiple: the 2-byte path), and entries naming blocks outside the cache,
    which the kernel skips (called through the C ABI: the Python wrapper passes entries through unchecked, as the
    reference does)."""
    kv = _kv((3, 2, 6, 32, 1, 4), 81)
    kv_d = kv.to(DEV)
    entries = [(0, 5, 17), (2, 1, 32), (-1, 3, 4), (4, 7, 4), (3, 4, 5)]
    pairs = torch.tensor(entries, dtype=torch.int32, device=DEV)
    lib = _lib.load()
    _lib.check(lib.vox_copy_kv_block_prefix(kv_d.data_ptr(), 6, 6, 32, 4, 2, pairs.data_ptr(), len(entries), 32,
                                            _lib.stream_handle(kv_d.device)), "copy")
    torch.cuda.synchronize()
    kvcopy.copy_kv_block_prefix(kv, [e for e in entries if 0 <= e[0] < 6 and 0 <= e[1] < 6])
    assert torch.equal(kv_d.cpu(), kv)
