"""Build + ctypes binding of ``oracle/mxfp4_ref.c`` (test infrastructure only).

The library is compiled with gcc into ``oracle/_build/`` by ``build()``, which
``__graft_entry__.build()`` calls; the tests load it with ``load()``.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "mxfp4_ref.c"
OUT = HERE / "_build" / "liboracle_mxfp4.so"

_lib = None


def build(force: bool = True) -> Path:
    if OUT.exists() and not force:
        return OUT
    OUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-std=c11",
                    str(SRC), "-o", str(tmp), "-lm"], check=True)
    tmp.replace(OUT)
    return OUT


def load():
    global _lib
    if _lib is None:
        if not OUT.exists():
            build()
        lib = ctypes.CDLL(str(OUT))
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        lib.oracle_decode_f32.argtypes = [p, p, i64, i64, p]
        lib.oracle_decode_f32.restype = None
        lib.oracle_decode_f64.argtypes = [p, p, i64, i64, p]
        lib.oracle_decode_f64.restype = None
        lib.oracle_matvec_seqfma.argtypes = [p, p, p, i64, i64, i64, p]
        lib.oracle_matvec_seqfma.restype = None
        _lib = lib
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def decode_f32(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    n, kh = packed.shape
    out = np.empty((n, kh * 2), dtype=np.float32)
    load().oracle_decode_f32(_ptr(packed), _ptr(scales), n, kh * 2, _ptr(out))
    return out


def decode_f64(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """float64 decode, bit-identical to ``decode_f32(...).astype(float64)``; the ctypes call
    releases the GIL, so threads decode experts in parallel."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    n, kh = packed.shape
    if scales.shape != (n, kh * 2 // 32):
        raise ValueError(f"scales shape {scales.shape} does not match packed {packed.shape}")
    out = np.empty((n, kh * 2), dtype=np.float64)
    load().oracle_decode_f64(_ptr(packed), _ptr(scales), n, kh * 2, _ptr(out))
    return out


def matvec_seqfma(x: np.ndarray, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.uint8)
    m, k = x.shape
    n = packed.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    load().oracle_matvec_seqfma(_ptr(x), _ptr(packed), _ptr(scales), m, n, k, _ptr(out))
    return out
