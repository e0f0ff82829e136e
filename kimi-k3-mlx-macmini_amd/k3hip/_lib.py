"""ctypes binding of libk3hip.so (the C-ABI declared in include/k3hip.h).

There is no fallback: if the library is missing or cannot be loaded, every k3hip entry
point raises ``K3LibraryError``.  Status codes from the C-ABI become the exception types
the reference raises for the same conditions (``ValueError`` for shape / scale-range
problems, as ``air_llm/kernels/metal/mxfp4_matvec.py:85-86`` and
``air_llm/models/kimi_k3/mxfp4.py:63-65`` do).
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libk3hip.so")

K3_OK, K3_ERR_SHAPE, K3_ERR_DTYPE, K3_ERR_ALIGN, K3_ERR_SCALE_RANGE = 0, 1, 2, 3, 4
K3_ERR_WORKSPACE, K3_ERR_HIP, K3_ERR_NULL = 5, 6, 7

K3_F32, K3_BF16 = 0, 1
K3_ACT_SILU, K3_ACT_SITU = 0, 1
K3_ROUTE_SOFTMAX, K3_ROUTE_SIGMOID_BIAS = 0, 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float

# name -> argtypes (restype is int unless listed in _RESTYPE)
SIGNATURES: dict[str, list] = {
    "k3_last_error": [],
    "k3_version": [],
    "k3_mxfp4_decode": [_P, _P, _P, _I32, _I64, _I64, _P],
    "k3_scale_minmax": [_P, _I64, _P, _P],
    "k3_mxfp4_matvec": [_P, _I32, _P, _P, _P, _I32, _I64, _I64, _I64, _P],
    "k3_expert_ffn_workspace_size": [_I64],
    "k3_expert_ffn": [_P, _I32, _P, _P, _P, _P, _P, _P, _P, _I32, _I64, _I64, _I32, _F32, _F32,
                      _P, _I64, _P],
    "k3_expert_ffn_noalloc": [_P, _I32, _P, _P, _P, _P, _P, _P, _P, _I32, _I64, _I64, _I32, _F32, _F32, _P],
    "k3_moe_layer_workspace_size": [_I64, _I64, _I64, _I64, _I64],
    "k3_moe_layer_workspace_offsets": [_I64, _I64, _I64, _I64, _I64, _P],
    "k3_moe_route": [_P, _I32, _P, _P, _I32, _I32, _F32, _I64, _I64, _I64, _P, _I64, _P],
    "k3_moe_topk": [_P, _I64, _I64, _I64, _P, _I32, _I32, _F32, _I64, _P, _P, _P, _P, _P],
    "k3_moe_layer_decode": [_P, _I32, _P, _P, _I32, _I32, _F32, _P, _P, _P, _P, _P, _I32, _I64, _I64,
                            _I64, _I64, _I64, _I32, _F32, _F32, _P, _I64, _P],
    "k3_moe_latent_layer_workspace_size": [_I64, _I64, _I64, _I64, _I64, _I64],
    "k3_moe_latent_layer_decode": [_P, _I32, _P, _P, _I32, _F32, _P, _P, _P, _P, _F32, _P, _P, _P, _P, _I32, _I64, _I64,
                                   _I64, _I64, _I64, _I64, _I32, _F32, _F32, _P, _I64, _P],
    "k3_mla_workspace_size": [_I64, _I64],
    "k3_mla_decode_absorbed": [_P, _P, _I64, _I64, _I32, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64,
                               _I64, _I64, _F32, _P, _I32, _I64, _P, _I64, _P],
    "k3_mla_decode_absorbed_f32": [_P, _P, _I64, _I64, _I32, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64,
                                   _I64, _I64, _F32, _P, _I32, _I64, _P, _I64, _P],
    "k3_mla_step_workspace_size": [_I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64],
    "k3_mla_step_decode": [_P, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _F32,
                           _F32, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P],
    "k3_kda_recurrent_decode": [_P, _P, _P, _P, _P, _I32, _P, _P, _I32, _I64, _I64, _I64, _I64, _F32, _P],
    "k3_kda_recurrent": [_P, _P, _P, _P, _P, _I32, _P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _F32, _P],
    "k3_kda_step_workspace_size": [_I64],
    "k3_kda_step_decode": [_P, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32,
                           _I64, _I64, _I64, _I64, _F32, _F32, _P, _I64, _P],
    "k3_moe_grouped_workspace_size": [_I64, _I64, _I64, _I64, _I64],
    "k3_moe_grouped_ffn": [_P, _I32, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I32, _F32, _F32,
                           _P, _I64, _P],
    "k3_moe_routed_workspace_size": [_I64, _I64, _I64, _I64, _I64],
    "k3_moe_routed_decode": [_P, _I32, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I32, _F32, _F32,
                             _P, _I64, _P],
    "k3_moe_layer_multi_workspace_size": [_I64, _I64, _I64, _I64, _I64, _I64],
    "k3_moe_layer_multi_workspace_offsets": [_I64, _I64, _I64, _I64, _I64, _I64, _P],
    "k3_moe_layer_decode_multi": [_P, _I32, _P, _P, _I32, _I32, _F32, _P, _P, _P, _P, _P, _I32, _I64, _I64,
                                  _I64, _I64, _I64, _I64, _I32, _F32, _F32, _P, _I64, _P],
    "k3_moe_latent_layer_multi_workspace_size": [_I64, _I64, _I64, _I64, _I64, _I64, _I64],
    "k3_moe_latent_layer_multi_workspace_offsets": [_I64, _I64, _I64, _I64, _I64, _I64, _I64, _P],
    "k3_moe_latent_layer_decode_multi": [_P, _I32, _P, _P, _I32, _F32, _P, _P, _P, _P, _F32, _P, _P, _P, _P, _I32,
                                         _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _F32, _F32, _P, _I64, _P],
    "k3_stream_read": [_P, _I64, _P, _P],
    "k3_stream_copy": [_P, _P, _I64, _P],
}
_RESTYPE = {"k3_last_error": ctypes.c_char_p, "k3_version": ctypes.c_char_p,
            "k3_expert_ffn_workspace_size": ctypes.c_int64,
            "k3_moe_layer_workspace_size": ctypes.c_int64,
            "k3_moe_latent_layer_workspace_size": ctypes.c_int64,
            "k3_mla_workspace_size": ctypes.c_int64,
            "k3_mla_step_workspace_size": ctypes.c_int64,
            "k3_kda_step_workspace_size": ctypes.c_int64,
            "k3_moe_grouped_workspace_size": ctypes.c_int64,
            "k3_moe_routed_workspace_size": ctypes.c_int64,
            "k3_moe_layer_multi_workspace_size": ctypes.c_int64,
            "k3_moe_latent_layer_multi_workspace_size": ctypes.c_int64}


class K3LibraryError(ImportError):
    """libk3hip.so is not built or cannot be loaded."""


_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise K3LibraryError(
                        f"{LIB_PATH} is not built; run `python kimi-k3-mlx-macmini_amd/build.py` "
                        "(or __graft_entry__.build()).  There is no CPU fallback.")
                try:
                    h = ctypes.CDLL(str(LIB_PATH))
                except OSError as e:  # pragma: no cover - depends on the ROCm install
                    raise K3LibraryError(f"cannot load {LIB_PATH}: {e}") from e
                for name, args in SIGNATURES.items():
                    fn = getattr(h, name)
                    fn.argtypes = args
                    fn.restype = _RESTYPE.get(name, ctypes.c_int)
                _lib = h
    return _lib


def call(name: str, *args) -> None:
    """Call a k3_* entry point and turn a nonzero status into an exception."""
    rc = getattr(lib(), name)(*args)
    if rc != K3_OK:
        msg = lib().k3_last_error().decode(errors="replace")
        if rc in (K3_ERR_SHAPE, K3_ERR_SCALE_RANGE, K3_ERR_ALIGN, K3_ERR_WORKSPACE, K3_ERR_NULL):
            raise ValueError(msg)
        if rc == K3_ERR_DTYPE:
            raise TypeError(msg)
        raise RuntimeError(msg)


def exported_symbols() -> list[str]:
    return sorted(SIGNATURES)
