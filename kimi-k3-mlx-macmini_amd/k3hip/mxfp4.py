"""MXFP4 format helpers on MI355X -- the counterpart of air_llm/models/kimi_k3/mxfp4.py.

Same names and argument meaning as the reference module; ``*_mlx`` aliases are kept so
callers written against the reference resolve unchanged.

Format (``mxfp4.py:3-11``): low nibble = element 2i, high nibble = element 2i+1; bit 3 is
the sign, bits 0-2 index [0, .5, 1, 1.5, 2, 3, 4, 6]; one E8M0 byte ``2**(b-127)`` per 32
elements along the input axis.  Decoding is bit-exact with ``k3ref/weights.py:29-37`` for
every code and every scale byte (including byte 0's subnormal, where the Metal path
flushes to zero, ``mxfp4.py:47-53``).
"""
from __future__ import annotations

import torch

from . import _lib
from . import _torch as T

E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
GROUP = 32


def decode_scale(scales: torch.Tensor) -> torch.Tensor:
    """E8M0 bytes -> float32 ``2**(b-127)`` (``mxfp4.py:41-55``).  Byte 0 gives the
    subnormal 2**-127 (bit pattern 0x00400000), byte 255 gives +inf."""
    b = scales.to(torch.int32)
    bits = torch.where(b == 0, torch.full_like(b, 0x00400000), b << 23)
    return bits.view(torch.float32)


decode_scale_mlx = decode_scale


def assert_scales_representable(scales: torch.Tensor) -> None:
    """Raise ValueError unless every E8M0 byte is in 2..252 (``mxfp4.py:58-65``).

    Runs as one device reduction; the two resulting bytes are the only device->host copy.
    """
    T.require_device(scales)
    s = scales.contiguous()
    mm = torch.empty(2, dtype=torch.int32, device=s.device)
    _lib.call("k3_scale_minmax", T.ptr(s), s.numel(), T.ptr(mm), T.stream(s))
    lo, hi = (int(v) for v in mm.tolist())
    if s.numel() and (lo < 2 or hi > 252):
        raise ValueError(f"Unsupported MXFP4 scale range {lo}..{hi}; require 2..252 "
                         "to avoid subnormal scales, overflow, and E8M0 NaN")


def _check_pair(packed: torch.Tensor, scales: torch.Tensor, group_size: int):
    if packed.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise TypeError("packed and scales must be uint8")
    if group_size != GROUP:
        raise ValueError(f"group_size {group_size} unsupported; the format fixes 32")
    if packed.dim() != 2 or scales.dim() != 2:
        raise ValueError("packed [N, K/2] and scales [N, K/32] must be 2-D")
    n, kh = packed.shape
    if kh * 2 % GROUP or tuple(scales.shape) != (n, kh * 2 // GROUP):
        raise ValueError(f"scales shape {tuple(scales.shape)} does not match packed "
                         f"{tuple(packed.shape)} (expected ({n}, {kh * 2 // GROUP}))")


def decode_mxfp4(packed: torch.Tensor, scales: torch.Tensor, group_size: int = GROUP,
                 out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """packed [R, C/2] u8, scales [R, C/32] u8 -> [R, C] out_dtype (``mxfp4.py:68-81``)."""
    _check_pair(packed, scales, group_size)
    T.require_device(packed, scales)
    packed = T.contiguous_aligned(packed)
    scales = scales.contiguous()
    n, kh = packed.shape
    out = torch.empty((n, kh * 2), dtype=out_dtype, device=packed.device)
    _lib.call("k3_mxfp4_decode", T.ptr(packed), T.ptr(scales), T.ptr(out),
              T.dtype_code(out_dtype), n, kh * 2, T.stream(packed))
    return out


decode_mxfp4_mlx = decode_mxfp4


def mxfp4_matvec(x: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor,
                 group_size: int = GROUP, accum_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """The reference's unfused definition (``mxfp4.py:84-92``): decode W to bf16 on the
    GPU, then ``x.bf16 @ W.T`` through the BLAS library, result in ``accum_dtype``.
    Slower and looser than the fused kernel; kept as the ``fused=False`` path."""
    w = decode_mxfp4(packed, scales, group_size, out_dtype=torch.bfloat16)
    return (x.to(torch.bfloat16) @ w.T).to(accum_dtype)
