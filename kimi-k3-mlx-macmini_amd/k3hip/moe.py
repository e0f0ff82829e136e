"""MoE expert FFN on MI355X -- the counterpart of LatentMoE.expert_forward
(air_llm/models/kimi_k3/moe.py:90-103, k3ref/layers.py:226-234).

``expert_ffn_fused(x, gate, up, down)`` runs one expert (``gate``/``up``/``down`` are the
``(packed, scales)`` pairs an ``expert_source`` returns) in a single persistent HIP launch
at batch 1: gate and up rows are reduced by the same wave so ``act = f(gate, up)`` never
round-trips, and the down projection's weights stream while the grid waits for ``act``.
"""
from __future__ import annotations

import torch

from . import _lib, _workspace
from . import _torch as T

ACTS = {"silu": _lib.K3_ACT_SILU, "swiglu": _lib.K3_ACT_SILU, "situ": _lib.K3_ACT_SITU}


def _act_code(act: str) -> int:
    try:
        return ACTS[act]
    except KeyError:
        raise ValueError(f"unknown activation {act!r}; expected one of {sorted(ACTS)}") from None


def expert_ffn_fused(x: torch.Tensor, gate, up, down, act: str = "silu", beta: float = 1.0,
                     linear_beta: float | None = None,
                     out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """One expert at batch 1: x [1, H] or [H] -> [1, H] (or [H])."""
    squeeze = x.dim() == 1
    x2 = x.reshape(1, -1) if squeeze else x
    if x2.shape[0] != 1:
        raise ValueError("expert_ffn_fused is the batch-1 kernel; use expert_ffn for M > 1")
    (gp, gs), (upk, us), (dp, ds) = gate, up, down
    H = x2.shape[1]
    I = gp.shape[0]
    if gp.shape[1] * 2 != H or upk.shape != gp.shape or tuple(dp.shape) != (H, I // 2):
        raise ValueError(f"expert shapes do not match: x {tuple(x2.shape)}, gate {tuple(gp.shape)}, "
                         f"up {tuple(upk.shape)}, down {tuple(dp.shape)}")
    T.require_device(x2, gp, gs, upk, us, dp, ds)
    if x2.dtype not in (torch.float32, torch.bfloat16):
        x2 = x2.to(torch.float32)
    x2 = T.contiguous_aligned(x2)
    gp, upk, dp = (T.contiguous_aligned(t) for t in (gp, upk, dp))
    gs, us, ds = (t.contiguous() for t in (gs, us, ds))
    ws_bytes = int(_lib.lib().k3_expert_ffn_workspace_size(I))
    ws = _workspace.get(x2.device, ws_bytes, "expert_ffn")
    out = torch.empty((1, H), dtype=out_dtype, device=x2.device)
    _lib.call("k3_expert_ffn", T.ptr(x2), T.dtype_code(x2.dtype), T.ptr(gp), T.ptr(gs), T.ptr(upk),
              T.ptr(us), T.ptr(dp), T.ptr(ds), T.ptr(out), T.dtype_code(out_dtype), H, I,
              _act_code(act), float(beta), float(linear_beta or 0.0), T.ptr(ws), ws.numel(),
              T.stream(x2))
    return out.reshape(-1) if squeeze else out
