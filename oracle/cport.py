"""ctypes front end of ``pkv_oracle.c`` -- TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg.  ``build()`` compiles the C restatement with gcc into
``oracle/libpkv_oracle.so``; ``load()`` loads it (building it when absent).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "pkv_oracle.c"
LIBRARY = HERE / "libpkv_oracle.so"

_lib = None


def build(verbose=False):
    """Compile the C oracle (gcc -O2 -fopenmp, strict IEEE float arithmetic)."""
    command = ["gcc", "-O2", "-fPIC", "-shared", "-fopenmp", "-fno-fast-math",
               "-ffp-contract=off", "-std=c11", str(SOURCE), "-o", str(LIBRARY) + ".tmp", "-lm"]
    if verbose:
        print(" ".join(command))
    subprocess.run(command, check=True)
    os.replace(str(LIBRARY) + ".tmp", LIBRARY)
    return LIBRARY


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY.exists():
        build()
    lib = ctypes.CDLL(str(LIBRARY))
    c_p = ctypes.c_void_p
    lib.pkvo_f32_to_f16.argtypes = [ctypes.c_float]
    lib.pkvo_f32_to_f16.restype = ctypes.c_uint16
    lib.pkvo_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.pkvo_f16_to_f32.restype = ctypes.c_float
    lib.pkvo_quantize_rows.argtypes = [c_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, c_p, c_p, c_p]
    lib.pkvo_quantize_rows.restype = None
    lib.pkvo_paged_attention.argtypes = (
        [c_p] + [ctypes.c_int] * 9 + [c_p, ctypes.c_int, c_p, c_p, c_p] + [c_p] * 8
        + [ctypes.c_float, c_p, ctypes.c_int])
    lib.pkvo_paged_attention.restype = ctypes.c_int
    _lib = lib
    return lib


def _ptr(array):
    return None if array is None else array.ctypes.data_as(ctypes.c_void_p)


def quantize_rows(values, bits, group_size):
    """Reference-format ``(codes, scale f16, bias f16)`` of ``values [..., D]``."""
    lib = load()
    x = np.ascontiguousarray(values, np.float32)
    dim = x.shape[-1]
    rows = int(np.prod(x.shape[:-1]))
    padded = (dim + group_size - 1) // group_size * group_size
    codes = np.empty(x.shape[:-1] + (padded * bits // 8,), np.uint8)
    scale = np.empty(x.shape[:-1] + (padded // group_size,), np.float16)
    bias = np.empty_like(scale)
    lib.pkvo_quantize_rows(_ptr(x), rows, dim, bits, group_size, _ptr(codes), _ptr(scale),
                           _ptr(bias))
    return codes, scale, bias


def paged_attention(queries, block_table, lengths, positions, widths, *, heads_kv, page_tokens,
                    bits, group_size=32, pages=None, float_pages=None, float_f16=False,
                    scale, threads=0):
    """Causal GQA attention over reference-format pages; float32 ``[B,H,Q,D]``.

    ``pages`` = ``(kc [N,HK,P,Dq], ks [N,HK,P,NG], kb, vc, vs, vb)`` for quantized
    pages, ``float_pages`` = ``(k [N,HK,P,D], v)`` as uint16 bits for float pages.
    """
    lib = load()
    q = np.ascontiguousarray(queries, np.float32)
    batch, heads, width, dim = q.shape
    table = np.ascontiguousarray(block_table, np.int32)
    lengths = np.ascontiguousarray(lengths, np.int32)
    positions = np.ascontiguousarray(positions, np.int32)
    widths = np.ascontiguousarray(widths, np.int32)
    out = np.zeros(q.shape, np.float32)
    if bits:
        arrays = [np.ascontiguousarray(a) for a in pages] + [None, None]
    else:
        arrays = [None] * 6 + [np.ascontiguousarray(a).view(np.uint16) for a in float_pages]
    lib.pkvo_paged_attention(
        _ptr(q), batch, heads, heads_kv, width, dim, page_tokens, bits or 0, group_size,
        int(float_f16), _ptr(table), table.shape[1], _ptr(lengths), _ptr(positions),
        _ptr(widths), *[_ptr(a) for a in arrays], float(scale), _ptr(out), int(threads))
    return out
