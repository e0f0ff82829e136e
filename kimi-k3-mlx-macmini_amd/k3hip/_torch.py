"""Torch tensor plumbing for the C-ABI: device pointers, dtype enums and streams."""
from __future__ import annotations

import ctypes

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.K3_F32, torch.bfloat16: _lib.K3_BF16}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise TypeError(f"unsupported dtype {dt}; k3hip takes float32 or bfloat16") from None


def ptr(t: torch.Tensor | None):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream(t: torch.Tensor):
    """The current HIP stream of t's device, as a void*."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_device(*ts: torch.Tensor) -> None:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"k3hip kernels take device tensors; got {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")


def contiguous_aligned(t: torch.Tensor) -> torch.Tensor:
    """Row-contiguous with a 16-byte aligned base (the 128-bit load paths need it);
    the counterpart of ensure_row_contiguous=True (mxfp4_matvec.py:71)."""
    if not t.is_contiguous():
        t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t
