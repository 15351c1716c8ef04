"""ctypes binding of libpkv.so (the C ABI in include/pkv.h).

The library is the only compute path of this package: when it is missing or
fails to load, every call raises ``NativeLibraryMissing`` -- there is no CPU
fallback.  Tensors are torch device tensors; their data pointers and the
current HIP stream are passed through the C ABI.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "libpkv.so"

PKV_OK, PKV_INVALID_ARGUMENT, PKV_UNSUPPORTED, PKV_OUT_OF_MEMORY, PKV_LAUNCH_FAILED = range(5)

# Every symbol include/pkv.h declares, with ctypes signatures.
_c_p, _i32, _i64, _f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float


class Layout(ctypes.Structure):
    """``pkv_layout`` (include/pkv.h)."""

    _fields_ = [("num_kv_heads", _i32), ("head_dim", _i32), ("page_tokens", _i32),
                ("bits", _i32), ("group_size", _i32), ("float_kind", _i32)]


_LP = ctypes.POINTER(Layout)

SIGNATURES = {
    "pkv_version": ([], ctypes.c_int),
    "pkv_last_error": ([], ctypes.c_char_p),
    "pkv_page_bytes": ([_LP], _i64),
    "pkv_stored_dim": ([_LP], _i32),
    "pkv_append_quantize": ([_c_p, _LP, _c_p, _i64, _c_p, _c_p, _i32, _i32, _c_p, _i32, _c_p,
                             _c_p, _c_p], ctypes.c_int),
    "pkv_paged_attention": ([_c_p, _LP, _c_p, _i64, _c_p, _i32, _i32, _i32, _c_p, _i32, _c_p,
                             _c_p, _c_p, _f32, _i32, _c_p, _i64, _c_p], ctypes.c_int),
    "pkv_paged_attention_noalloc": ([_c_p, _LP, _c_p, _i64, _c_p, _i32, _i32, _i32, _c_p, _i32,
                                     _c_p, _c_p, _c_p, _f32, _i32, _c_p], ctypes.c_int),
    "pkv_append_paged_attention": ([_c_p, _LP, _c_p, _i64, _c_p, _c_p, _c_p, _i32, _i32, _c_p,
                                    _i32, _c_p, _f32, _i32, _c_p, _i64, _c_p], ctypes.c_int),
    "pkv_select_decode_kernel": ([ctypes.c_int], ctypes.c_int),
    "pkv_attention_waves": ([_LP, _i32, _i32], _i32),
    "pkv_attention_default_waves": ([_LP, _i32, _i32, _i32], _i32),
    "pkv_attention_workspace_bytes": ([_LP, _i32, _i32, _i32], _i64),
    "pkv_gather_pages": ([_c_p, _LP, _c_p, _i64, _c_p, _i32, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p],
                         ctypes.c_int),
    "pkv_copy_pages": ([_c_p, _LP, _c_p, _i64, _c_p, _c_p, _i32], ctypes.c_int),
    "pkv_read_probe": ([_c_p, _LP, _c_p, _i64, _c_p, _i64, _i32, _c_p], ctypes.c_int),
    "pkv_quantize_rows": ([_c_p, _c_p, _i64, _i32, _i32, _i32, _i32, _c_p, _c_p, _c_p],
                          ctypes.c_int),
    "pkv_dequantize_rows": ([_c_p, _c_p, _c_p, _c_p, _i64, _i32, _i32, _i32, _c_p],
                            ctypes.c_int),
    "pkv_rope_qkv": ([_c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32, _c_p, _c_p, _c_p, _c_p,
                      _c_p], ctypes.c_int),
    "pkv_arena_state_bytes": ([_i32], _i64),
    "pkv_arena_init": ([_c_p, _c_p, _i32], ctypes.c_int),
    "pkv_arena_reserve": ([_c_p, _c_p, _i32, _i32, _c_p, _i32, _i32, _c_p, _c_p, _c_p, _i32,
                           _c_p, _i32, _i64, _c_p, _c_p, _c_p], ctypes.c_int),
    "pkv_arena_truncate": ([_c_p, _c_p, _i32, _i32, _c_p, _i32, _i32, _c_p, _c_p, _c_p, _i32],
                           ctypes.c_int),
    "pkv_arena_fork": ([_c_p, _c_p, _i32, _i32, _c_p, _i32, _i32, _c_p, _c_p, _c_p, _i32],
                       ctypes.c_int),
}


class NativeLibraryMissing(RuntimeError):
    """libpkv.so is absent or unloadable: the paged path has no other backend."""


class NativeError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


_lock = threading.Lock()
_lib = None


def load(path=None):
    """Load libpkv.so and bind every exported symbol (idempotent)."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = Path(path) if path else LIBRARY
        if not target.exists():
            raise NativeLibraryMissing(
                f"{target} is not built; run `python -m pkv.build` (hipcc, gfx950)")
        try:
            lib = ctypes.CDLL(str(target))
        except OSError as exc:
            raise NativeLibraryMissing(f"cannot load {target}: {exc}") from exc
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes, fn.restype = args, res
        if path is None:
            _lib = lib
        return lib


def last_error():
    return load().pkv_last_error().decode(errors="replace")


def check(code, what):
    """Map a libpkv status to the reference's exception types."""
    if code == PKV_OK:
        return
    message = f"{what}: {last_error()}"
    from pkv.cache_errors import CacheCapacityError
    from pkv.modes import ModelCapabilityUnsupported

    if code == PKV_INVALID_ARGUMENT:
        raise ValueError(message)
    if code == PKV_UNSUPPORTED:
        raise ModelCapabilityUnsupported(message)
    if code == PKV_OUT_OF_MEMORY:
        raise CacheCapacityError(message)
    raise NativeError(code, message)


def ptr(tensor):
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def stream_handle(device=None):
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
