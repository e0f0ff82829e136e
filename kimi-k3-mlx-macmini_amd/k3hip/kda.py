"""Kimi Delta Attention recurrence on MI355X -- the counterpart of
``KDAAttention._recurrent`` (air_llm/models/kimi_k3/attention_kda.py:65-90).

``kda_recurrent(q, k, v, g, beta, scale, state)`` takes the reference's tensors
(q, k [B, T, H, K]; v [B, T, HV, V]; g [B, T, HV, K] log decay; beta [B, T, HV]; state
[B, HV, K, V] or None) and returns ``(o [B, T, HV, V] fp32, state [B, HV, K, V] fp32)``.
Each token is one launch of ``k3_kda_recurrent_decode`` over all B * HV heads, updating the
fp32 state in place (the reference allocates a new state per step).  A state passed in is
used as the output state when it is a contiguous fp32 device tensor, else copied once.
"""
from __future__ import annotations

import torch

from . import _lib
from . import _torch as T


def kda_recurrent(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                  scale: float | None = None, state: torch.Tensor | None = None):
    T.require_device(q, k, v, g, beta, state)
    if q.dim() != 4 or k.shape != q.shape or v.dim() != 4 or g.dim() != 4 or beta.dim() != 3:
        raise ValueError("q, k [B, T, H, K], v [B, T, HV, V], g [B, T, HV, K], beta [B, T, HV] expected")
    B, Tn, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    if tuple(v.shape[:2]) != (B, Tn) or tuple(g.shape) != (B, Tn, HV, K) or tuple(beta.shape) != (B, Tn, HV):
        raise ValueError(f"shape mismatch: q {tuple(q.shape)}, v {tuple(v.shape)}, g {tuple(g.shape)}, "
                         f"beta {tuple(beta.shape)}")
    if HV % H:
        raise ValueError(f"value heads {HV} must be a multiple of q/k heads {H}")
    if scale is None:
        scale = K ** -0.5
    dt = torch.bfloat16 if all(t.dtype == torch.bfloat16 for t in (q, k, v, g, beta)) else torch.float32
    # time-major, so each step's [B, heads, dim] slice is contiguous
    q, k, v, g, beta = (t.to(dt).transpose(0, 1).contiguous() for t in (q, k, v, g, beta))
    if state is None:
        S = torch.zeros((B, HV, K, V), dtype=torch.float32, device=q.device)
    elif tuple(state.shape) != (B, HV, K, V):
        raise ValueError(f"state must be [{B}, {HV}, {K}, {V}]; got {tuple(state.shape)}")
    elif state.dtype == torch.float32 and state.is_contiguous() and state.data_ptr() % 16 == 0:
        S = state
    else:
        S = state.to(torch.float32).contiguous().clone()
    o = torch.empty((Tn, B, HV, V), dtype=torch.float32, device=q.device)
    code = T.dtype_code(dt)
    st = T.stream(q)
    for i in range(Tn):
        # B sequences are B * HV independent heads: q/k head b * H + h serves value heads
        # (b * HV + h * G) .. + G, the same grouping as within one sequence
        _lib.call("k3_kda_recurrent_decode", T.ptr(q[i]), T.ptr(k[i]), T.ptr(v[i]), T.ptr(g[i]), T.ptr(beta[i]),
                  code, T.ptr(S), T.ptr(o[i]), _lib.K3_F32, B * H, B * HV, K, V, float(scale), st)
    return o.transpose(0, 1), S
