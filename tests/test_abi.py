"""C-ABI checks that need no GPU: the library loads, exports every entry point that
include/k3hip.h declares, and the binding table matches the header."""
from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "k3hip.h"


def declared_entry_points() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(k3_[a-z0-9_]+)\s*\(", text))


def test_header_declares_entry_points():
    names = declared_entry_points()
    assert {"k3_mxfp4_decode", "k3_mxfp4_matvec", "k3_last_error"} <= names


def test_library_exports_every_declared_symbol():
    from k3hip import _lib
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} missing: run __graft_entry__.build() first")
    h = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared_entry_points() if not hasattr(h, n)]
    assert not missing, missing


def test_binding_table_matches_header():
    from k3hip import _lib
    assert set(_lib.SIGNATURES) == declared_entry_points()


def test_version_and_error_string_callable_without_gpu():
    from k3hip import _lib
    lib = _lib.lib()
    assert lib.k3_version().startswith(b"k3hip")
    assert isinstance(lib.k3_last_error(), bytes)


def test_argument_validation_without_gpu():
    """Status codes for bad arguments are produced on the host before any launch."""
    from k3hip import _lib
    lib = _lib.lib()
    p = ctypes.c_void_p(16)
    s = ctypes.c_void_p(0)
    # K not a multiple of 32
    assert lib.k3_mxfp4_matvec(p, 1, p, p, p, 0, 1, 8, 48, s) == _lib.K3_ERR_SHAPE
    assert b"multiple of 32" in lib.k3_last_error()
    # bad dtype enum
    assert lib.k3_mxfp4_matvec(p, 7, p, p, p, 0, 1, 8, 64, s) == _lib.K3_ERR_DTYPE
    # null pointer
    assert lib.k3_mxfp4_decode(None, p, p, 0, 8, 64, s) == _lib.K3_ERR_NULL
    # misaligned x
    assert lib.k3_mxfp4_matvec(ctypes.c_void_p(18), 1, p, p, p, 0, 1, 8, 64, s) == _lib.K3_ERR_ALIGN
    with pytest.raises(ValueError, match="multiple of 32"):
        _lib.call("k3_mxfp4_matvec", p, 1, p, p, p, 0, 1, 8, 48, s)
    with pytest.raises(TypeError):
        _lib.call("k3_mxfp4_matvec", p, 7, p, p, p, 0, 1, 8, 64, s)


def test_step_and_recurrence_validation_without_gpu():
    """The MLA step, KDA recurrence and KDA step entry points reject bad arguments on the
    host (null pointers, dtypes, shapes, aliasing) before any launch."""
    from k3hip import _lib
    lib = _lib.lib()
    p, s = ctypes.c_void_p(256), ctypes.c_void_p(0)
    # KDA recurrence: null state, bad dtype, key_dim != 128, value_dim not a multiple of 32
    assert lib.k3_kda_recurrent(p, p, p, p, p, 0, None, p, 0, 4, 2, 2, 128, 128, 0.1, s) == _lib.K3_ERR_NULL
    assert lib.k3_kda_recurrent(p, p, p, p, p, 9, p, p, 0, 4, 2, 2, 128, 128, 0.1, s) == _lib.K3_ERR_DTYPE
    assert lib.k3_kda_recurrent(p, p, p, p, p, 0, p, p, 0, 4, 2, 2, 64, 128, 0.1, s) == _lib.K3_ERR_SHAPE
    assert lib.k3_kda_recurrent_decode(p, p, p, p, p, 0, p, p, 0, 2, 2, 128, 48, 0.1, s) == _lib.K3_ERR_SHAPE
    assert lib.k3_kda_recurrent(p, p, p, p, p, 0, p, p, 0, 4, 3, 4, 128, 128, 0.1, s) == _lib.K3_ERR_SHAPE
    # KDA step: conv_in and conv_out must differ; head_dim must be 128
    args = [p, 1] + [p] * 17 + [p, 0, 1024, 8, 128, 4, -5.0, 1e-5, p, 1 << 30, s]
    bad = list(args)
    bad[13] = bad[14] = ctypes.c_void_p(4096)
    assert lib.k3_kda_step_decode(*bad) == _lib.K3_ERR_SHAPE and b"distinct" in lib.k3_last_error()
    bad = list(args)
    bad[23] = 64
    assert lib.k3_kda_step_decode(*bad) == _lib.K3_ERR_SHAPE
    bad = list(args)
    bad[2] = None
    assert lib.k3_kda_step_decode(*bad) == _lib.K3_ERR_NULL
    # MLA step: position outside the cache, widths above the limit
    margs = [p, 1] + [p] * 9 + [p, 512, p, 64, 256, 256, 1e-5, 0.1, p, 0, 1024, 512, 8, 128, 64, 128, 512, p, 1 << 30, s]
    assert lib.k3_mla_step_decode(*margs) == _lib.K3_ERR_SHAPE and b"outside the cache" in lib.k3_last_error()
    m2 = list(margs)
    m2[16], m2[21] = 0, 20000
    assert lib.k3_mla_step_decode(*m2) == _lib.K3_ERR_SHAPE
