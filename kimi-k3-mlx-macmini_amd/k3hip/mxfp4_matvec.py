"""Fused MXFP4 matvec on MI355X -- the counterpart of
air_llm/kernels/metal/mxfp4_matvec.py (``mxfp4_matvec_fused``, ``expert_projection``).

``mxfp4_matvec_fused(x, packed, scales)`` keeps the reference signature and contract:
x ``[M, K]``, packed ``[N, K/2]`` u8, scales ``[N, K/32]`` u8, output ``[M, N]`` float32,
``ValueError`` on a K mismatch (``mxfp4_matvec.py:75-96``).  The reference casts x to
float32; here bf16 x is consumed as bf16 (its float32 value is the same number, and the
products with the exact E2M1 x 2**e weights are exact either way), other float dtypes
are cast to float32.  ``out_dtype=torch.bfloat16`` returns the round-to-nearest-even of
the float32 accumulator instead.
"""
from __future__ import annotations

import torch

from . import _lib
from . import _torch as T


def _prep_x(x: torch.Tensor) -> torch.Tensor:
    if x.dtype not in (torch.float32, torch.bfloat16):
        x = x.to(torch.float32)
    return T.contiguous_aligned(x)


def mxfp4_matvec_fused(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor,
                       out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """y = x @ W.T with W given by (packed, scales); fp32 accumulation."""
    if x.dim() != 2:
        raise ValueError(f"x must be [M, K]; got shape {tuple(x.shape)}")
    M = x.shape[0]
    N = packed.shape[0]
    if packed.shape[1] * 2 != x.shape[1]:
        raise ValueError(f"K mismatch: x has {x.shape[1]}, packed implies {packed.shape[1] * 2}")
    if packed.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise TypeError("packed and scales must be uint8")
    if tuple(scales.shape) != (N, x.shape[1] // 32) or x.shape[1] % 32:
        raise ValueError(f"scales shape {tuple(scales.shape)} does not match K={x.shape[1]}")
    T.require_device(x, packed, scales)
    x = _prep_x(x)
    packed = T.contiguous_aligned(packed)
    scales = scales.contiguous()
    out = torch.empty((M, N), dtype=out_dtype, device=x.device)
    _lib.call("k3_mxfp4_matvec", T.ptr(x), T.dtype_code(x.dtype), T.ptr(packed), T.ptr(scales), T.ptr(out),
              T.dtype_code(out_dtype), M, N, x.shape[1], T.stream(x))
    return out


def expert_projection(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """Shape convention of ``mxfp4_matvec.py:99-105``: 1-D x in, 1-D y out."""
    squeeze = x.dim() == 1
    if squeeze:
        x = x.reshape(1, -1)
    y = mxfp4_matvec_fused(x, packed, scales)
    return y.reshape(-1) if squeeze else y
