"""Exact, fast float16 matmul for the oracle (test infrastructure).

``matmul16(a, b)`` returns what NumPy's own ``a @ b`` returns for float16 operands
(float32 accumulation in increasing k, one rounding to float16; see halfmm.c) but
runs as a blocked multi-threaded C loop instead of NumPy's scalar one, which makes
the reference's float16 path affordable at the benchmark configs. The shared library
is compiled from ``oracle/halfmm.c`` on first use into ``oracle/_lib/`` (git-ignored).
When no compiler is available ``matmul16`` falls back to NumPy itself.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "halfmm.c")
LIB = os.path.join(HERE, "_lib", "libhalfmm.so")
_lib = None
_tried = False


def build(force: bool = False) -> str | None:
    """Compile halfmm.c (gcc, OpenMP, AVX2/FMA/F16C). Returns the library path."""
    if not force and os.path.exists(LIB) and os.path.getmtime(LIB) >= os.path.getmtime(SRC):
        return LIB
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    tmp = LIB + f".tmp{os.getpid()}"
    cmd = ["gcc", "-O3", "-fPIC", "-shared", "-fopenmp", "-mavx2", "-mfma", "-mf16c",
           SRC, "-o", tmp]
    try:
        subprocess.run(cmd, check=True, capture_output=True)
    except (OSError, subprocess.CalledProcessError):
        return None
    os.replace(tmp, LIB)
    return LIB


def _load():
    global _lib, _tried
    if _tried:
        return _lib
    _tried = True
    path = build()
    if path is None:
        return None
    lib = C.CDLL(path)
    lib.halfmm.restype = C.c_int
    lib.halfmm.argtypes = [C.c_void_p, C.c_long, C.c_long, C.c_void_p, C.c_long, C.c_long,
                           C.c_void_p, C.c_long, C.c_long, C.c_long, C.c_long, C.c_long]
    _lib = lib
    return lib


def available() -> bool:
    return _load() is not None


def _mm2(lib, a, b, out):
    es = 2
    M, K = a.shape
    N = b.shape[1]
    if M == 0 or N == 0:
        return
    if K == 0:
        out[...] = 0
        return
    rc = lib.halfmm(a.ctypes.data, a.strides[0] // es, a.strides[1] // es,
                    b.ctypes.data, b.strides[0] // es, b.strides[1] // es,
                    out.ctypes.data, out.strides[0] // es, out.strides[1] // es, M, N, K)
    if rc != 0:
        raise MemoryError("halfmm: out of memory")


def matmul16(a, b):
    """``a @ b`` for float16 arrays (2-D, or equal leading batch dims / a 2-D ``b``)."""
    a = np.asarray(a)
    b = np.asarray(b)
    if a.dtype != np.float16 or b.dtype != np.float16:
        raise TypeError("matmul16 takes float16 operands")
    lib = _load()
    if lib is None or a.ndim < 2 or b.ndim < 2:
        return a @ b
    if any(s % 2 for s in a.strides + b.strides):
        return a @ b
    if a.ndim == 2 and b.ndim == 2:
        out = np.empty((a.shape[0], b.shape[1]), dtype=np.float16)
        _mm2(lib, a, b, out)
        return out
    if b.ndim == 2:  # (..., M, K) @ (K, N): fold the batch into rows when a is dense
        lead = a.shape[:-2]
        a2 = np.ascontiguousarray(a).reshape(-1, a.shape[-1])
        out = np.empty((a2.shape[0], b.shape[1]), dtype=np.float16)
        _mm2(lib, a2, b, out)
        return out.reshape(*lead, a.shape[-2], b.shape[1])
    if a.shape[:-2] != b.shape[:-2]:
        return a @ b
    lead = a.shape[:-2]
    a3 = a.reshape(-1, *a.shape[-2:])
    b3 = b.reshape(-1, *b.shape[-2:])
    out = np.empty((a3.shape[0], a.shape[-2], b.shape[-1]), dtype=np.float16)
    for i in range(a3.shape[0]):
        _mm2(lib, a3[i], b3[i], out[i])
    return out.reshape(*lead, a.shape[-2], b.shape[-1])
