"""Dense projections on the BLAS library (hipBLASLt through torch) for the multi-token paths.

``mm_f32(a, w)`` is ``a @ w.T`` with fp32 output, exact products and fp32 accumulation for
bf16 or fp32 ``a`` against bf16 or fp32 ``w``, without copying the weight:

* bf16 ``a``, bf16 ``w``: one GEMM with fp32 output;
* fp32 ``a``, bf16 ``w``: ``a`` is the exact sum of three bf16 terms (8 + 8 + 8 significant
  bits), each one GEMM with fp32 output, summed;
* fp32 ``w``: an fp32 GEMM.

This is the arithmetic of the reference's fp32 router and of MLX's promotion of a bf16
weight against an fp32 activation (``air_llm/models/kimi_k3/moe.py:67-68``).

``mm_ref(a, w)`` keeps the reference's dtype promotion instead: operands of one dtype give
that dtype (a bf16 GEMM returns bf16, as MLX's bf16 matmul does), mixed operands give fp32.
The paths that restate the reference's own unfused definitions use it.
"""
from __future__ import annotations

import torch


def bf16_terms(a: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Three bf16 tensors whose fp32 sum is exactly ``a`` (fp32) for normal values."""
    t1 = a.to(torch.bfloat16)
    r = a - t1.float()
    t2 = r.to(torch.bfloat16)
    t3 = (r - t2.float()).to(torch.bfloat16)
    return t1, t2, t3


def _mm_bf16_f32(a2: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return torch.mm(a2, w.t(), out_dtype=torch.float32)


def mm_f32(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """a [..., K] @ w[N, K]^T -> fp32 [..., N] with exact products and fp32 accumulation."""
    lead = a.shape[:-1]
    a2 = a.reshape(-1, a.shape[-1])
    if w.dtype == torch.float32:
        out = a2.to(torch.float32) @ w.t()
    elif w.dtype == torch.bfloat16:
        if a2.dtype == torch.bfloat16:
            out = _mm_bf16_f32(a2, w)
        else:
            t1, t2, t3 = bf16_terms(a2.to(torch.float32))
            out = _mm_bf16_f32(t1, w)
            out += _mm_bf16_f32(t2, w)
            out += _mm_bf16_f32(t3, w)
    else:
        raise TypeError(f"weights must be float32 or bfloat16; got {w.dtype}")
    return out.reshape(*lead, w.shape[0])


def mm_ref(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """a @ w.T with the reference's (MLX's) dtype promotion: same dtype in, same dtype out;
    bf16 against fp32 gives fp32."""
    if a.dtype == w.dtype:
        return a @ w.t()
    return mm_f32(a, w)
