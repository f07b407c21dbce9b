"""Copy the first n token slots of KV-cache blocks in every causal layer's K and V, in one launch, with the
reference's interface (reference: nanovllm_voxcpm/kernels/kv_copy.py:31-41; callers model/runner.py:232-248,
model/engine.py:383-452).

``copy_kv_block_prefix(kv, entries)``: kv is the engine's contiguous [layers, 2, blocks, block_size, kv_heads,
head_dim] cache, entries a list of (src block, dst block, n tokens). n is clipped to block_size and entries with
n <= 0 are dropped, as in the reference; the entries go to the GPU through a pinned buffer on the current stream and
one HIP kernel copies every entry's run in every plane (csrc/kv_copy.hip). Bit-exact.
"""

from __future__ import annotations

import torch

from .. import _lib


def copy_kv_block_prefix(kv: torch.Tensor, entries: list[tuple[int, int, int]]) -> None:
    assert kv.is_contiguous()
    layers, kvs, blocks, block_size = kv.shape[:4]
    entries = [(s, d, min(n, block_size)) for s, d, n in entries if n > 0]
    if not entries:
        return
    if kv.device.type != "cuda":
        raise ValueError(f"copy_kv_block_prefix: kv must be on a GPU, got {kv.device}")
    if kv.element_size() != 2:
        raise TypeError(f"copy_kv_block_prefix: 16-bit cache elements, got {kv.dtype}")
    per_token = kv.shape[4] * kv.shape[5]
    pairs = torch.tensor(entries, dtype=torch.int32, pin_memory=True).to(kv.device, non_blocking=True)
    lib = _lib.load()
    _lib.check(lib.vox_copy_kv_block_prefix(kv.data_ptr(), layers * kvs, blocks, block_size, per_token, 2,
                                            pairs.data_ptr(), len(entries), max(n for _, _, n in entries),
                                            _lib.stream_handle(kv.device)),
               "copy_kv_block_prefix")
