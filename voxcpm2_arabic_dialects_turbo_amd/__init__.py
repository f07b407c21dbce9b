"""MI355X-native (gfx950) paged-KV attention for the VoxCPM2 engine.

A drop-in for the reference engine's attention path (reference: nanovllm_voxcpm/model/layers.py:266-362 and the
context of nanovllm_voxcpm/engine/utils.py:25-99): ``Attention`` with the same constructor, attributes and
``forward(q, k, v)`` dispatch over the module-global ``Context``, backed by three HIP kernels in libvoxattn.so
(KV slot scatter, varlen GQA prefill on bf16 MFMA, split-KV paged decode) reached through a C ABI
(include/vox_attn.h). Build the library with ``python -m voxcpm2_arabic_dialects_turbo_amd.build``.
"""

from .context import Context, get_context, reset_context, set_context
from .layers import Attention
from .ops import (flash_attn_func, flash_attn_varlen_func, flash_attn_with_kvcache, store_kvcache, decode_attention,
                  varlen_attention)

__all__ = [
    "Attention",
    "Context",
    "get_context",
    "set_context",
    "reset_context",
    "store_kvcache",
    "flash_attn_varlen_func",
    "flash_attn_with_kvcache",
    "flash_attn_func",
    "decode_attention",
    "varlen_attention",
]
