"""Kimi Delta Attention on MI355X -- the counterpart of ``KDAAttention``
(air_llm/models/kimi_k3/attention_kda.py:32-115).

``KDAAttention(cfg, w)`` keeps the reference constructor, weight names and
``__call__(x, state=None, conv=None) -> (out, state, (cq, ck, cv))``.  Up to
``PREFILL_TOKENS`` tokens per call, every token of every sequence is one
``k3_kda_step_decode`` (projections, short convolutions, norms, gate, recurrence, gated
RMSNorm, o_proj in four launches); longer calls take ``prefill``: GEMMs over all tokens on
the BLAS library and the recurrence over all tokens in one ``k3_kda_recurrent`` launch.  The recurrent state is fp32
[B, H, 128, 128], updated in place; the convolution states come back as fp32 [B, k-1, C].

``kda_recurrent(q, k, v, g, beta, scale, state)`` takes the reference's tensors
(q, k [B, T, H, K]; v [B, T, HV, V]; g [B, T, HV, K] log decay; beta [B, T, HV]; state
[B, HV, K, V] or None) and returns ``(o [B, T, HV, V] fp32, state [B, HV, K, V] fp32)``.
All tokens are one launch of ``k3_kda_recurrent`` over all B * HV heads, the state kept in
registers between tokens and updated in place once (the reference allocates a new state
per step).  A state passed in is
used as the output state when it is a contiguous fp32 device tensor, else copied once.
"""
from __future__ import annotations

import torch

from . import _lib, _workspace
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
    # B sequences are B * HV independent heads: q/k head b * H + h serves value heads
    # (b * HV + h * G) .. + G, the same grouping as within one sequence; all tokens in one
    # launch, the state kept in registers between them
    _lib.call("k3_kda_recurrent", T.ptr(q), T.ptr(k), T.ptr(v), T.ptr(g), T.ptr(beta), code, T.ptr(S), T.ptr(o),
              _lib.K3_F32, Tn, B * H, B * HV, K, V, float(scale), st)
    return o.transpose(0, 1), S


class KDAAttention:
    """Drop-in for KDAAttention (attention_kda.py:32-115) on bf16 projection weights."""

    KEYS = ("q_proj.weight", "k_proj.weight", "v_proj.weight", "g_proj.weight",
            "o_proj.weight", "q_conv1d.weight", "k_conv1d.weight", "v_conv1d.weight",
            "f_a_proj.weight", "f_b_proj.weight", "b_proj.weight", "o_norm.weight",
            "A_log", "dt_bias")

    def __init__(self, cfg, w: dict):
        self.cfg = cfg
        H, D, K = cfg.kda_num_heads, cfg.kda_head_dim, cfg.kda_conv_size
        self.H, self.D, self.K = H, D, K
        bf = lambda n: T.contiguous_aligned(w[n].to(torch.bfloat16))  # noqa: E731
        f32 = lambda n: T.contiguous_aligned(w[n].to(torch.float32))  # noqa: E731
        self.q_w, self.k_w, self.v_w = bf("q_proj.weight"), bf("k_proj.weight"), bf("v_proj.weight")
        self.g_w, self.o_w = bf("g_proj.weight"), bf("o_proj.weight")
        self.fa, self.fb, self.b_w = bf("f_a_proj.weight"), bf("f_b_proj.weight"), bf("b_proj.weight")
        self.qc, self.kc, self.vc = (f32(n).reshape(H * D, K) for n in ("q_conv1d.weight", "k_conv1d.weight",
                                                                         "v_conv1d.weight"))
        self.o_norm_w, self.dt_bias = f32("o_norm.weight"), f32("dt_bias").reshape(-1)
        A = f32("A_log").reshape(-1)
        if A.shape[0] != D or (A.shape[0] > H and float(A[H:].abs().max()) != 0.0):
            raise ValueError("A_log must be [head_dim] with zeros past num_heads (attention_kda.py:50-54)")
        self.A_log = A

    def decode_step(self, x1, state, conv_in, conv_out, out) -> None:
        """One token of one sequence: x1 [hidden], state [H, D, D] fp32 (in place),
        conv_in / conv_out [3, k-1, H*D] fp32, out [hidden] fp32."""
        c = self.cfg
        nbytes = int(_lib.lib().k3_kda_step_workspace_size(self.H))
        ws = _workspace.get(x1.device, nbytes, "kda_step")
        _lib.call("k3_kda_step_decode", T.ptr(x1), T.dtype_code(x1.dtype), T.ptr(self.q_w), T.ptr(self.k_w),
                  T.ptr(self.v_w), T.ptr(self.g_w), T.ptr(self.o_w), T.ptr(self.fa), T.ptr(self.fb), T.ptr(self.b_w),
                  T.ptr(self.qc), T.ptr(self.kc), T.ptr(self.vc), T.ptr(conv_in), T.ptr(conv_out),
                  T.ptr(self.o_norm_w), T.ptr(self.A_log), T.ptr(self.dt_bias), T.ptr(state), T.ptr(out),
                  _lib.K3_F32, x1.shape[-1], self.H, self.D, self.K, float(c.kda_gate_lower_bound),
                  float(c.rms_norm_eps), T.ptr(ws), ws.numel(), T.stream(x1))

    PREFILL_TOKENS = 8   # more tokens per call than this take the prefill path

    @staticmethod
    def _mm(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """a [M, K] @ w[N, K]^T with fp32 output on the BLAS library.  A bf16 a (the layer
        input) meets the bf16 weight directly, with fp32 accumulation and output where torch
        offers it; an fp32 a (an intermediate) keeps its precision: fp32 operands."""
        if a.dtype == torch.bfloat16:
            try:
                return torch.mm(a, w.t(), out_dtype=torch.float32)
            except (RuntimeError, TypeError):
                pass
        return a.to(torch.float32) @ w.to(torch.float32).t()

    def prefill(self, x: torch.Tensor, state: torch.Tensor | None = None, conv: tuple | None = None):
        """Many tokens (attention_kda.py:94-115): the projections as GEMMs over all tokens
        (each weight read once), the convolutions, norms and gates as tensor ops, the
        recurrence over every token in one k3_kda_recurrent launch, the gated RMSNorm, and
        o_proj as one GEMM."""
        c = self.cfg
        B, Tn, hid = x.shape
        H, D, K = self.H, self.D, self.K
        P = H * D
        xf = x.reshape(B * Tn, hid)
        proj = lambda w: self._mm(xf, w).reshape(B, Tn, -1)  # noqa: E731
        outs, states = [], []
        for m, (w, cw) in enumerate(((self.q_w, self.qc), (self.k_w, self.kc), (self.v_w, self.vc))):
            y = proj(w)
            pad = (torch.zeros((B, K - 1, P), dtype=torch.float32, device=x.device) if conv is None
                   else conv[m].to(torch.float32).reshape(B, K - 1, P))
            xp = torch.cat([pad, y], dim=1)
            z = sum(cw[:, j] * xp[:, j:j + Tn] for j in range(K))
            outs.append(z * torch.sigmoid(z))
            states.append(xp[:, Tn:].contiguous())
        q, k, v = (o_.reshape(B, Tn, H, D) for o_ in outs)
        q = q * torch.rsqrt((q * q).sum(-1, keepdim=True) + 1e-6)
        k = k * torch.rsqrt((k * k).sum(-1, keepdim=True) + 1e-6)
        g_raw = self._mm(self._mm(xf, self.fa), self.fb).reshape(B, Tn, H, D) + self.dt_bias.reshape(H, D)
        g = c.kda_gate_lower_bound * torch.sigmoid(torch.exp(self.A_log[:H]).reshape(H, 1) * g_raw)
        beta = torch.sigmoid(proj(self.b_w))
        o, state = kda_recurrent(q, k, v, g, beta, D ** -0.5, state)
        og = proj(self.g_w).reshape(B, Tn, H, D)
        o = o * torch.rsqrt((o * o).mean(-1, keepdim=True) + c.rms_norm_eps) * self.o_norm_w * torch.sigmoid(og)
        out = self._mm(o.reshape(B * Tn, P), self.o_w).reshape(B, Tn, hid)
        return out, state, tuple(states)

    def __call__(self, x: torch.Tensor, state: torch.Tensor | None = None, conv: tuple | None = None):
        T.require_device(x, state)
        B, Tn, hid = x.shape
        if Tn > self.PREFILL_TOKENS:
            return self.prefill(x, state, conv)
        H, D, K = self.H, self.D, self.K
        P = H * D
        if state is None:
            state = torch.zeros((B, H, D, D), dtype=torch.float32, device=x.device)
        elif tuple(state.shape) != (B, H, D, D):
            raise ValueError(f"state must be [{B}, {H}, {D}, {D}]; got {tuple(state.shape)}")
        elif not (state.dtype == torch.float32 and state.is_contiguous() and state.data_ptr() % 16 == 0):
            state = state.to(torch.float32).contiguous().clone()
        bufs = [torch.zeros((B, 3, K - 1, P), dtype=torch.float32, device=x.device) for _ in range(2)]
        if conv is not None:
            for m in range(3):
                bufs[0][:, m] = conv[m].to(torch.float32).reshape(B, K - 1, P)
        xin = x if x.dtype in (torch.float32, torch.bfloat16) else x.to(torch.float32)
        xin = xin.contiguous()
        out = torch.empty((B, Tn, hid), dtype=torch.float32, device=x.device)
        for t in range(Tn):
            cin, cout = bufs[t % 2], bufs[(t + 1) % 2]
            for b in range(B):
                x1 = T.contiguous_aligned(xin[b, t])
                self.decode_step(x1, state[b], cin[b], cout[b], out[b, t])
        fin = bufs[Tn % 2]
        return out, state, (fin[:, 0], fin[:, 1], fin[:, 2])
