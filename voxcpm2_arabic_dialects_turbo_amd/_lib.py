"""ctypes bindings of libvoxattn.so (the C ABI declared in include/vox_attn.h).

The library must be built in-tree first (``python -m voxcpm2_arabic_dialects_turbo_amd.build``); there is no
fallback of any kind: a missing library raises. torch is imported before the library is opened so that the HIP
runtime torch loaded (libamdhip64.so.7) is the one libvoxattn.so binds to by SONAME, and the stream handles torch
hands out are valid in the library.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded before the library: shared HIP runtime)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libvoxattn.so")

VOX_OK, VOX_EINVAL, VOX_EHIP = 0, 1, 2
ABI_VERSION = 13

PLAN_NONE, PLAN_RECORD, PLAN_REUSE = 0, 1, 2

# every symbol include/vox_attn.h declares
EXPORTS = (
    "vox_last_error",
    "vox_abi_version",
    "vox_store_kvcache",
    "vox_decode_attn",
    "vox_decode_attn_store",
    "vox_decode_attn_noalloc",
    "vox_decode_workspace_bytes",
    "vox_decode_workgroups",
    "vox_set_decode_workgroups",
    "vox_prefill_attn",
    "vox_prefill_workspace_bytes",
    "vox_prefill_attn_store",
    "vox_prefill_attn_store_paged",
    "vox_prefill_attn_int8",
    "vox_prefill_attn_int8_store",
    "vox_prefill_int8_workspace_bytes",
    "vox_copy_kv_block_prefix",
)

_c_void_p, _i32, _i64, _f32, _size = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t

_SIGNATURES = {
    "vox_last_error": (ctypes.c_char_p, []),
    "vox_abi_version": (_i32, []),
    "vox_store_kvcache": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _i64,
                                 _i32, _i32, _c_void_p]),
    "vox_decode_attn": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i32, _c_void_p, _i64, _i32,
                               _c_void_p, _i32, _i32, _i32, _i32, _f32, _i32, _c_void_p, _size, _c_void_p,
                               _c_void_p]),
    "vox_decode_attn_store": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _c_void_p, _c_void_p,
                                     _c_void_p, _i64, _i32, _c_void_p, _i64, _i32, _c_void_p, _i32, _i32, _i32, _i32,
                                     _f32, _i32, _c_void_p, _size, _c_void_p, _c_void_p]),
    "vox_decode_attn_noalloc": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i32, _c_void_p, _i64, _i32,
                                       _c_void_p, _i32, _i32, _i32, _i32, _f32, _c_void_p, _c_void_p]),
    "vox_decode_workspace_bytes": (_size, [_i32]),
    "vox_decode_workgroups": (_i32, []),
    "vox_set_decode_workgroups": (None, [_i32]),
    "vox_prefill_attn": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64,
                                _i32, _c_void_p, _i64, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i32,
                                _i32, _i32, _f32, _i32, _c_void_p, _i64, _i32, _c_void_p, _size, _c_void_p]),
    "vox_prefill_workspace_bytes": (_size, [_i32]),
    "vox_prefill_attn_store": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _c_void_p, _c_void_p,
                                      _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i32, _f32,
                                      _i32, _c_void_p, _i64, _c_void_p]),
    "vox_prefill_attn_store_paged": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _c_void_p, _i64,
                                            _c_void_p, _c_void_p, _i64, _i32, _c_void_p, _i64, _i32, _c_void_p,
                                            _c_void_p, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _c_void_p, _i64,
                                            _i32, _c_void_p, _size, _c_void_p]),
    "vox_prefill_attn_int8_store": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _c_void_p, _i64,
                                           _c_void_p, _c_void_p, _i64, _i32, _c_void_p, _i64, _i32, _c_void_p,
                                           _c_void_p, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _c_void_p,
                                           _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _size, _c_void_p]),
    "vox_copy_kv_block_prefix": (_i32, [_c_void_p, _i64, _i64, _i32, _i64, _i32, _c_void_p, _i32, _i32, _c_void_p]),
    "vox_prefill_attn_int8": (_i32, [_c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64,
                                     _i32, _c_void_p, _i64, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i32,
                                     _i32, _i32, _f32, _i32, _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _c_void_p,
                                     _size, _c_void_p]),
    "vox_prefill_int8_workspace_bytes": (_size, [_i64, _i32, _i32, _i32, _i32, _i32, _i32]),
}


class VoxAttnError(RuntimeError):
    """The library rejected a call (VOX_EINVAL) or the HIP runtime failed a launch (VOX_EHIP)."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Opens libvoxattn.so once per process and declares every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise VoxAttnError(
                    f"{LIB_PATH} is not built: run `python -m voxcpm2_arabic_dialects_turbo_amd.build` "
                    "(hipcc, gfx950). There is no non-HIP fallback."
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.vox_abi_version() != ABI_VERSION:
                raise VoxAttnError(f"libvoxattn ABI {lib.vox_abi_version()} != {ABI_VERSION}: rebuild the library")
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status == VOX_OK:
        return
    msg = load().vox_last_error().decode(errors="replace")
    if status == VOX_EINVAL:
        raise ValueError(f"{what}: {msg}")
    raise VoxAttnError(f"{what}: {msg}")


def stream_handle(device: torch.device) -> int:
    """The hipStream_t of torch's current stream on ``device`` (0 = null stream)."""
    return torch.cuda.current_stream(device).cuda_stream


_capture_info = None


def capture_id(stream: int) -> int:
    """The id of the HIP graph capture in progress on ``stream``, 0 when it is not capturing
    (hipStreamGetCaptureInfo of the HIP runtime libvoxattn.so is linked against)."""
    global _capture_info
    if _capture_info is None:
        fn = load().hipStreamGetCaptureInfo
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_ulonglong)]
        _capture_info = fn
    status, ident = ctypes.c_int(0), ctypes.c_ulonglong(0)
    if _capture_info(stream, ctypes.byref(status), ctypes.byref(ident)) != 0:
        raise VoxAttnError("hipStreamGetCaptureInfo failed")
    return int(ident.value) if status.value == 1 else 0  # hipStreamCaptureStatusActive


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
