"""MoE expert FFN on MI355X -- the counterpart of LatentMoE.expert_forward
(air_llm/models/kimi_k3/moe.py:90-103, k3ref/layers.py:226-234).

``expert_ffn_fused(x, gate, up, down)`` runs one expert (``gate``/``up``/``down`` are the
``(packed, scales)`` pairs an ``expert_source`` returns) at batch 1 in two stream-ordered HIP
launches: gate and up rows are reduced by the same wave, which applies the activation and
writes ``act`` (fp32) to a workspace; the down projection is the batch-1 MXFP4 GEMV on it.
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


# ----------------------------------------------------------------------- routed layer

from dataclasses import dataclass  # noqa: E402
from typing import Callable  # noqa: E402

from . import _blas  # noqa: E402

ROUTES = {"softmax": _lib.K3_ROUTE_SOFTMAX, "sigmoid_bias": _lib.K3_ROUTE_SIGMOID_BIAS}
_DENSE_DTYPES = (torch.bfloat16, torch.float32)


@dataclass
class RouterResult:
    """Same fields as the reference's RouterResult (air_llm/models/kimi_k3/moe.py:32-37)."""
    expert_indices: torch.Tensor      # [N, top_k] int64, largest weight first
    expert_weights: torch.Tensor      # [N, top_k] float32
    raw_scores: torch.Tensor          # [N, num_experts] softmax probabilities / sigmoid scores
    corrected_scores: torch.Tensor    # raw + e_score_correction_bias (== raw for softmax)


@dataclass
class MoEConfig:
    """The config fields the routed layer reads (names follow K3Config,
    air_llm/models/kimi_k3/config.py), plus the router / activation choice."""
    hidden_size: int
    moe_intermediate_size: int
    num_experts: int
    num_experts_per_token: int
    shared_intermediate_size: int = 0
    moe_renormalize: bool = True
    routed_scaling_factor: float = 1.0
    router: str = "softmax"               # "softmax" (benchmark) | "sigmoid_bias" (K3)
    activation: str = "silu"              # "silu" (benchmark) | "situ" (K3)
    situ_beta: float = 1.0
    situ_linear_beta: float | None = None


def route_tokens(x: torch.Tensor, gate_w: torch.Tensor, bias: torch.Tensor | None, kind: int,
                 renormalize: bool, scaling: float, top_k: int) -> RouterResult:
    """Router + top-k for every token of x [..., H] (moe.py:65-76): the logits of all tokens
    as one GEMM with exact products and fp32 accumulation (the reference's fp32 router), then
    the selection for all tokens in one launch (k3_moe_topk)."""
    flat = x.reshape(-1, x.shape[-1])
    n, E = flat.shape[0], gate_w.shape[0]
    dev = gate_w.device
    idx = torch.empty((n, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((n, top_k), dtype=torch.float32, device=dev)
    scores = torch.empty((n, E), dtype=torch.float32, device=dev)
    corrected = torch.empty((n, E), dtype=torch.float32, device=dev)
    if n:
        logits = _blas.mm_f32(flat, gate_w).contiguous()
        _lib.call("k3_moe_topk", T.ptr(logits), E, n, E, T.ptr(bias), kind, int(bool(renormalize)),
                  float(scaling), top_k, T.ptr(idx), T.ptr(w), T.ptr(scores), T.ptr(corrected), T.stream(logits))
    return RouterResult(idx.to(torch.int64), w, scores, corrected)


def _dense(t: torch.Tensor | None, name: str) -> torch.Tensor | None:
    if t is not None and t.dtype not in _DENSE_DTYPES:
        raise TypeError(f"{name} must be bfloat16 (the checkpoint dtype) or float32 (validation mode); got {t.dtype}")
    return t


class RoutedMoE:
    """Drop-in for the routed path of LatentMoE (air_llm/models/kimi_k3/moe.py:40-132).

    ``RoutedMoE(cfg, layer, w, expert_source, fused=True)`` keeps the reference
    constructor: ``w`` holds ``gate.weight`` ([E, H]), optionally
    ``gate.e_score_correction_bias`` and ``shared_experts.{gate,up,down}_proj.weight``;
    ``expert_source(layer, expert, which)`` returns ``(packed, scales)`` device tensors for
    ``which`` in ``w1`` (gate), ``w3`` (up), ``w2`` (down).  Dense weights are bf16 (the
    checkpoint dtype) or fp32 (the reference loader's validation mode, loader.py:90-95).

    With ``fused=True`` and bf16 dense weights, every expert is made resident once (the
    source is called E x 3 times at build) and addressed through a device pointer table, so
    a decode step is three launches with no host synchronisation.  ``fused=False`` (or fp32
    dense weights) runs the reference's own structure instead: ``route``, then a host loop
    over the distinct routed experts with ``expert_forward`` built on ``_proj``, whose
    unfused form is the HIP decode to bf16 followed by a BLAS matmul (moe.py:79-88), and the
    shared expert with the reference's dtype promotion.
    """

    DECODE_TOKENS = 8  # up to this many tokens: decode kernels; more: grouped (prefill)

    def __init__(self, cfg, layer: int, w: dict, expert_source: Callable, fused: bool = True):
        self.cfg, self.L = cfg, layer
        self.src = expert_source
        self.fused = fused
        self.gate_w = _dense(w["gate.weight"], "gate.weight")
        self.gate_b = w.get("gate.e_score_correction_bias")
        self.sh_gate = _dense(w.get("shared_experts.gate_proj.weight"), "shared_experts.gate_proj.weight")
        self.sh_up = _dense(w.get("shared_experts.up_proj.weight"), "shared_experts.up_proj.weight")
        self.sh_down = _dense(w.get("shared_experts.down_proj.weight"), "shared_experts.down_proj.weight")
        self.device = self.gate_w.device
        if self.gate_b is not None:
            self.gate_b = self.gate_b.to(torch.float32).contiguous()
        dense = [self.gate_w] + [t for t in (self.sh_gate, self.sh_up, self.sh_down) if t is not None]
        # the fused decode kernels read bf16 router / shared rows
        self._fast = fused and all(t.dtype == torch.bfloat16 for t in dense)
        self._table = None
        self._keep = []

    # ------------------------------------------------------------------ helpers
    @property
    def _H(self):
        return self.gate_w.shape[1]

    @property
    def _E(self):
        return self.gate_w.shape[0]

    @property
    def _k(self):
        return int(self.cfg.num_experts_per_token)

    @property
    def _I(self):
        return int(self.cfg.moe_intermediate_size)

    @property
    def _Is(self):
        return 0 if self.sh_gate is None else self.sh_gate.shape[0]

    def _act(self):
        act = getattr(self.cfg, "activation", "silu")
        beta = float(getattr(self.cfg, "situ_beta", 1.0) or 1.0)
        lb = getattr(self.cfg, "situ_linear_beta", None)
        return act, beta, lb

    def _route_args(self):
        kind = ROUTES[getattr(self.cfg, "router", "softmax")]
        bias = self.gate_b if kind == _lib.K3_ROUTE_SIGMOID_BIAS else None
        return kind, bias

    def expert_table(self) -> torch.Tensor:
        """[E, 6] int64 device pointers, built once from expert_source."""
        if self._table is None:
            ptrs = []
            for e in range(self._E):
                row = []
                for which in ("w1", "w3", "w2"):
                    p, s = self.src(self.L, e, which)
                    p = T.contiguous_aligned(p)
                    s = s.contiguous()
                    T.require_device(p, s)
                    if p.device != self.device:
                        raise ValueError("experts must live on the router's device")
                    self._keep += [p, s]
                    row += [p.data_ptr(), s.data_ptr()]
                ptrs.append(row)
            self._table = torch.tensor(ptrs, dtype=torch.int64, device=self.device)
        return self._table

    def _workspace(self):
        nbytes = int(_lib.lib().k3_moe_layer_workspace_size(self._H, self._I, self._Is, self._E, self._k))
        return _workspace.get(self.device, nbytes, "moe_layer")

    def _records(self, ws: torch.Tensor) -> RouterResult:
        import ctypes
        off = (ctypes.c_int64 * 8)()
        _lib.call("k3_moe_layer_workspace_offsets", self._H, self._I, self._Is, self._E, self._k, off)
        E, k = self._E, self._k

        def f32(o, n):
            return ws[o:o + 4 * n].view(torch.float32).clone()

        idx = ws[off[3]:off[3] + 4 * k].view(torch.int32).to(torch.int64).reshape(1, k)
        return RouterResult(idx, f32(off[4], k).reshape(1, k), f32(off[1], E).reshape(1, E),
                            f32(off[2], E).reshape(1, E))

    def _x1(self, x):
        x1 = x.reshape(1, -1)
        if x1.dtype not in (torch.float32, torch.bfloat16):
            x1 = x1.to(torch.float32)
        return T.contiguous_aligned(x1)

    # ------------------------------------------------------------------ API
    def route(self, x: torch.Tensor) -> RouterResult:
        """Router + top-k for each token of x [..., H] (moe.py:65-76), on x as given."""
        kind, bias = self._route_args()
        return route_tokens(x, self.gate_w, bias, kind, bool(self.cfg.moe_renormalize),
                            float(self.cfg.routed_scaling_factor), self._k)

    def _proj(self, h: torch.Tensor, e: int, which: str) -> torch.Tensor:
        """h @ W.T for one MXFP4 projection of expert e (moe.py:79-88): fused, the MXFP4
        matvec (weights decoded in registers, fp32 out); unfused, the HIP decode to bf16
        then a BLAS matmul in h's dtype, as the reference's ``h @ decode(...).T.astype(h.dtype)``."""
        p, s = self.src(self.L, e, which)
        if h.dtype not in (torch.float32, torch.bfloat16):
            h = h.to(torch.float32)
        if self.fused:
            from .mxfp4_matvec import mxfp4_matvec_fused
            return mxfp4_matvec_fused(h, p, s)
        from .mxfp4 import decode_mxfp4
        return h @ decode_mxfp4(p, s, out_dtype=torch.bfloat16).t().to(h.dtype)

    def expert_forward(self, h: torch.Tensor, e: int) -> torch.Tensor:
        """One routed expert on h [N, H] (moe.py:90-103): gate and up projections, the
        activation in fp32, the down projection.  One fused token runs the two-launch expert
        kernel; otherwise the three projections go through ``_proj``."""
        act, beta, lb = self._act()
        if self.fused and h.shape[0] == 1:
            gate, up, down = (self.src(self.L, e, w) for w in ("w1", "w3", "w2"))
            return expert_ffn_fused(h, gate, up, down, act, beta, lb)
        g = self._proj(h, e, "w1")
        u = self._proj(h, e, "w3")
        return self._proj(_act_torch(g.float(), u.float(), act, beta, lb), e, "w2")

    def shared_forward(self, x: torch.Tensor) -> torch.Tensor:
        """Shared expert on the original hidden state (moe.py:105-107).  Fused: exact
        products with fp32 accumulation and fp32 intermediates on the BLAS library, no weight
        copy (inside a decode step it runs in the layer kernels).  Unfused: the reference's
        dtype promotion (a bf16 input against bf16 weights gives bf16 gate / up)."""
        act, beta, lb = self._act()
        mm = _blas.mm_f32 if self.fused else _blas.mm_ref
        g = mm(x, self.sh_gate)
        u = mm(x, self.sh_up)
        return mm(_act_torch(g.float(), u.float(), act, beta, lb), self.sh_down).float()

    def _combine_loop(self, h: torch.Tensor, r: RouterResult, width: int) -> torch.Tensor:
        """The reference's dispatch loop (moe.py:119-127): for each distinct routed expert,
        gather its tokens, run expert_forward, scale by the gate weight, scatter-add."""
        n = h.shape[0]
        y = torch.zeros((n, width), dtype=torch.float32, device=h.device)
        idx = r.expert_indices.tolist()   # drives host control flow, as np_indices does
        for e in sorted({v for row in idx for v in row}):
            tok = [t for t, row in enumerate(idx) if e in row]
            slot = [idx[t].index(e) for t in tok]
            ti = torch.tensor(tok, device=h.device)
            out = self.expert_forward(h[ti], e).float()
            wts = r.expert_weights[ti, torch.tensor(slot, device=h.device)].reshape(-1, 1)
            y.index_add_(0, ti, out * wts)
        return y

    def grouped_forward(self, x: torch.Tensor, router: RouterResult | None = None,
                        out_dtype=torch.float32) -> torch.Tensor:
        """Prefill form of __call__ for x [..., H]: route every token on x as given (or take
        the given RouterResult), then run the routed experts grouped by expert on the device
        (moe_grouped_ffn); the shared expert, if any, runs on the BLAS library."""
        return self._forward_routed(x, router, out_dtype, moe_grouped_ffn)

    def multi_forward(self, x: torch.Tensor, router: RouterResult | None = None,
                      out_dtype=torch.float32) -> torch.Tensor:
        """Decode form of __call__ for a few tokens x [..., H] (at most DECODE_TOKENS): route
        every token, then every expert any token selects runs once against all the tokens
        routed to it (moe_routed_decode: the union of the routed experts built on the device,
        fp32 accumulation); the shared expert, if any, runs on the BLAS library."""
        return self._forward_routed(x, router, out_dtype, moe_routed_decode)

    def _forward_routed(self, x, router, out_dtype, routed_fn, validate=None):
        """Routed experts by routed_fn plus the shared expert; a caller's RouterResult has its
        ids checked on the device (validate), the layer's own routing needs no check."""
        orig = x.shape
        flat = x.reshape(-1, orig[-1])
        if validate is None:
            validate = router is not None
        if router is None:
            router = self.route(flat)
        act, beta, lb = self._act()
        y = routed_fn(flat, router.expert_indices, router.expert_weights, self.expert_table(), self._I,
                      act, beta, lb, out_dtype=torch.float32, validate=validate)
        if self.sh_gate is not None:
            y = y + self.shared_forward(flat)
        return y.to(out_dtype).reshape(*orig[:-1], self._H)

    def __call__(self, x: torch.Tensor, return_router: bool = False, out_dtype=torch.float32):
        orig = x.shape
        flat = x.reshape(-1, orig[-1])
        if not self._fast:
            r = self.route(flat)
            y = self._combine_loop(flat, r, self._H)
            if self.sh_gate is not None:
                y = y + self.shared_forward(flat)
            y = y.to(out_dtype).reshape(*orig[:-1], self._H)
            return (y, r) if return_router else y
        if flat.shape[0] > self.DECODE_TOKENS:
            # many tokens: grouped GEMMs on MXFP4 MFMA, every routed expert read once per tile
            r = self.route(flat)
            y = self._forward_routed(flat, r, out_dtype, moe_grouped_ffn, validate=False)
            y = y.reshape(*orig[:-1], self._H)
            return (y, r) if return_router else y
        if flat.shape[0] > 1:
            return self._decode_multi(flat, orig, return_router, out_dtype)
        kind, bias = self._route_args()
        act, beta, lb = self._act()
        table = self.expert_table()
        outs, recs = [], []
        for t in range(flat.shape[0]):
            xt = self._x1(flat[t])
            ws = self._workspace()
            out = torch.empty((1, self._H), dtype=out_dtype, device=self.device)
            _lib.call("k3_moe_layer_decode", T.ptr(xt), T.dtype_code(xt.dtype), T.ptr(self.gate_w), T.ptr(bias),
                      kind, int(bool(self.cfg.moe_renormalize)), float(self.cfg.routed_scaling_factor),
                      T.ptr(table), T.ptr(self.sh_gate), T.ptr(self.sh_up), T.ptr(self.sh_down), T.ptr(out),
                      T.dtype_code(out_dtype), self._H, self._I, self._Is, self._E, self._k, ACTS[act],
                      float(beta), float(lb or 0.0), T.ptr(ws), ws.numel(), T.stream(xt))
            outs.append(out)
            if return_router:
                recs.append(self._records(ws))
        y = (outs[0] if len(outs) == 1 else torch.cat(outs)).reshape(*orig[:-1], self._H)
        if not return_router:
            return y
        r = RouterResult(*(torch.cat([getattr(rr, f) for rr in recs]) for f in
                           ("expert_indices", "expert_weights", "raw_scores", "corrected_scores")))
        return y, r


    def _decode_multi(self, flat, orig, return_router, out_dtype):
        """2..DECODE_TOKENS tokens in one pass (k3_moe_layer_decode_multi): router and
        shared expert on HIP row kernels, every routed expert any token selects read once for
        all the tokens routed to it; no host synchronisation.  The RouterResult comes from
        the workspace records."""
        import ctypes
        kind, bias = self._route_args()
        act, beta, lb = self._act()
        table = self.expert_table()
        n = flat.shape[0]
        x = flat if flat.dtype in (torch.float32, torch.bfloat16) else flat.to(torch.float32)
        x = T.contiguous_aligned(x)
        H, I, Is, E, k = self._H, self._I, self._Is, self._E, self._k
        nbytes = int(_lib.lib().k3_moe_layer_multi_workspace_size(n, H, I, Is, E, k))
        ws = _workspace.get(self.device, nbytes, "moe_layer_multi")
        out = torch.empty((n, H), dtype=out_dtype, device=self.device)
        _lib.call("k3_moe_layer_decode_multi", T.ptr(x), T.dtype_code(x.dtype), T.ptr(self.gate_w), T.ptr(bias),
                  kind, int(bool(self.cfg.moe_renormalize)), float(self.cfg.routed_scaling_factor), T.ptr(table),
                  T.ptr(self.sh_gate), T.ptr(self.sh_up), T.ptr(self.sh_down), T.ptr(out), T.dtype_code(out_dtype),
                  n, H, I, Is, E, k, ACTS[act], float(beta), float(lb or 0.0), T.ptr(ws), ws.numel(), T.stream(x))
        y = out.reshape(*orig[:-1], H)
        if not return_router:
            return y
        off = (ctypes.c_int64 * 5)()
        _lib.call("k3_moe_layer_multi_workspace_offsets", n, H, I, Is, E, k, off)

        def rec(o, count, dt):
            return ws[o:o + 4 * count].view(dt).clone()

        r = RouterResult(rec(off[3], n * k, torch.int32).to(torch.int64).reshape(n, k),
                         rec(off[4], n * k, torch.float32).reshape(n, k),
                         rec(off[1], n * E, torch.float32).reshape(n, E),
                         rec(off[2], n * E, torch.float32).reshape(n, E))
        return y, r


def _rmsnorm32(y: torch.Tensor, w32: torch.Tensor, eps: float) -> torch.Tensor:
    """KimiRMSNorm in fp32 (ops.py:11-14)."""
    y = y.float()
    return w32 * (y * torch.rsqrt((y * y).mean(dim=-1, keepdim=True) + eps))


class LatentMoE:
    """Drop-in for K3's routed layer, LatentMoE (air_llm/models/kimi_k3/moe.py:40-132).

    ``LatentMoE(cfg, layer, w, expert_source, fused=True)`` keeps the reference constructor
    and weight names: ``gate.weight`` [E, H] and ``gate.e_score_correction_bias`` [E]
    (sigmoid + bias routing), ``routed_expert_down_proj.weight`` [L, H] and
    ``routed_expert_up_proj.weight`` [H, L] (the latent projections),
    ``routed_expert_norm.weight`` [L], ``shared_experts.{gate,up,down}_proj.weight`` (K3's two
    shared experts are one MLP of twice the width).  Dense weights are bf16 (the checkpoint
    dtype) or fp32 (validation mode, loader.py:90-95).  ``expert_source(layer, e, which)``
    returns latent-width MXFP4 experts (gate/up [I, L], down [L, I]).  cfg carries the
    K3Config fields hidden_size, routed_expert_hidden_size, moe_intermediate_size,
    num_experts, num_experts_per_token, moe_renormalize, routed_scaling_factor, situ_beta,
    situ_linear_beta and rms_norm_eps.

    ``__call__(x)`` (moe.py:110-132): route on x; h = x W_down^T (bf16 for a bf16 x, as the
    reference's bf16 matmul gives; fp32 for an fp32 x); the routed experts (SiTU) on h;
    KimiRMSNorm of their weighted sum in fp32; the up projection in fp32; plus the shared
    expert on the original x.  With ``fused=True`` and bf16 dense weights, one token runs
    k3_moe_latent_layer_decode (four launches), 2..DECODE_TOKENS tokens
    k3_moe_latent_layer_decode_multi (eight launches, every selected expert read once for
    all its tokens) and more tokens run the routed experts grouped by expert
    (k3_moe_grouped_ffn); none synchronises with the host.  ``fused=False`` or fp32 dense
    weights run the reference's structure (``RoutedMoE`` describes it)."""

    DECODE_TOKENS = 8  # up to this many tokens: decode kernels; more: grouped

    def __init__(self, cfg, layer: int, w: dict, expert_source: Callable, fused: bool = True):
        self.cfg, self.L = cfg, layer
        self.fused = fused
        H = int(cfg.hidden_size)
        self.latent = int(getattr(cfg, "routed_expert_hidden_size"))
        rcfg = MoEConfig(hidden_size=H, moe_intermediate_size=int(cfg.moe_intermediate_size),
                         num_experts=int(cfg.num_experts), num_experts_per_token=int(cfg.num_experts_per_token),
                         moe_renormalize=bool(cfg.moe_renormalize),
                         routed_scaling_factor=float(cfg.routed_scaling_factor), router="sigmoid_bias",
                         activation="situ", situ_beta=float(cfg.situ_beta),
                         situ_linear_beta=getattr(cfg, "situ_linear_beta", None))
        shared = {f"shared_experts.{n}_proj.weight": w[f"shared_experts.{n}_proj.weight"]
                  for n in ("gate", "up", "down") if f"shared_experts.{n}_proj.weight" in w}
        self._routed = RoutedMoE(rcfg, layer, {"gate.weight": w["gate.weight"],
                                               "gate.e_score_correction_bias": w["gate.e_score_correction_bias"],
                                               **shared}, expert_source, fused)
        self.src = expert_source
        self.down = _dense(w["routed_expert_down_proj.weight"], "routed_expert_down_proj.weight")
        self.up = _dense(w["routed_expert_up_proj.weight"], "routed_expert_up_proj.weight")
        self.norm_w = w["routed_expert_norm.weight"]
        if tuple(self.down.shape) != (self.latent, H) or tuple(self.up.shape) != (H, self.latent):
            raise ValueError(f"latent projections must be [{self.latent}, {H}] and [{H}, {self.latent}]; got "
                             f"{tuple(self.down.shape)}, {tuple(self.up.shape)}")
        T.require_device(self.down, self.up, self.norm_w)
        self._norm32 = self.norm_w.float().contiguous()
        self._fast = (self._routed._fast and self.down.dtype == torch.bfloat16
                      and self.up.dtype == torch.bfloat16)

    def route(self, x: torch.Tensor) -> RouterResult:
        """Sigmoid + bias router on the hidden state (moe.py:65-76)."""
        return self._routed.route(x)

    def _proj(self, h: torch.Tensor, e: int, which: str) -> torch.Tensor:
        """h @ W.T for one MXFP4 projection of expert e, fused or unfused (moe.py:79-88)."""
        return self._routed._proj(h, e, which)

    def expert_forward(self, h: torch.Tensor, e: int) -> torch.Tensor:
        """One routed expert on latent rows h [N, L] (moe.py:90-103)."""
        return self._routed.expert_forward(h, e)

    def shared_forward(self, x: torch.Tensor) -> torch.Tensor:
        """Shared expert(s) on the original hidden state (moe.py:105-107)."""
        return self._routed.shared_forward(x)

    def __call__(self, x: torch.Tensor, return_router: bool = False, out_dtype=torch.float32):
        orig = x.shape
        flat = x.reshape(-1, orig[-1])
        if not self._fast:
            return self._forward_loop(flat, orig, return_router, out_dtype)
        if flat.shape[0] == 1:
            return self._decode(flat, orig, return_router, out_dtype)
        if flat.shape[0] <= self.DECODE_TOKENS:
            return self._decode_multi(flat, orig, return_router, out_dtype)
        return self.grouped_forward(flat, return_router, out_dtype, orig)

    def _forward_loop(self, flat, orig, return_router, out_dtype):
        """The reference's structure (moe.py:110-132) with ``fused`` choosing _proj's form."""
        c, R = self.cfg, self._routed
        r = self.route(flat)
        h = _blas.mm_ref(flat, self.down)                                  # hidden -> latent
        y = R._combine_loop(h, r, self.latent)
        y = _rmsnorm32(y, self._norm32, float(c.rms_norm_eps))
        y = _blas.mm_f32(y, self.up)                                       # latent -> hidden
        if R.sh_gate is not None:
            y = y + self.shared_forward(flat)
        y = y.to(out_dtype).reshape(*orig[:-1], orig[-1])
        return (y, r) if return_router else y

    def _decode(self, flat, orig, return_router, out_dtype):
        """One token: k3_moe_latent_layer_decode (route, latent down, routed experts,
        norm, up projection, shared experts; four launches, no host synchronisation)."""
        c, R = self.cfg, self._routed
        act, beta, lb = R._act()
        table = R.expert_table()
        H, Lw, I, Is, E, k = R._H, self.latent, R._I, R._Is, R._E, R._k
        nbytes = int(_lib.lib().k3_moe_latent_layer_workspace_size(H, Lw, I, Is, E, k))
        outs, recs = [], []
        for t in range(flat.shape[0]):
            xt = R._x1(flat[t])
            ws = _workspace.get(R.device, nbytes, "moe_latent")
            out = torch.empty((1, H), dtype=out_dtype, device=R.device)
            _lib.call("k3_moe_latent_layer_decode", T.ptr(xt), T.dtype_code(xt.dtype), T.ptr(R.gate_w),
                      T.ptr(R.gate_b), int(bool(c.moe_renormalize)), float(c.routed_scaling_factor), T.ptr(table),
                      T.ptr(self.down), T.ptr(self.up), T.ptr(self._norm32), float(c.rms_norm_eps), T.ptr(R.sh_gate),
                      T.ptr(R.sh_up), T.ptr(R.sh_down), T.ptr(out), T.dtype_code(out_dtype), H, Lw, I, Is, E, k,
                      ACTS[act], float(beta), float(lb or 0.0), T.ptr(ws), ws.numel(), T.stream(xt))
            outs.append(out)
            if return_router:
                recs.append(R._records(ws))
        y = (outs[0] if len(outs) == 1 else torch.cat(outs)).reshape(*orig[:-1], H)
        if not return_router:
            return y
        return y, RouterResult(*(torch.cat([getattr(rr, f) for rr in recs]) for f in
                                 ("expert_indices", "expert_weights", "raw_scores", "corrected_scores")))

    def _decode_multi(self, flat, orig, return_router, out_dtype):
        """2..DECODE_TOKENS tokens in one pass (k3_moe_latent_layer_decode_multi, eight
        launches, no host synchronisation): router, latent down, shared experts and the up
        projection on T-token HIP row kernels, every routed expert any token selects read
        once for all the tokens routed to it.  The RouterResult comes from the workspace."""
        import ctypes
        c, R = self.cfg, self._routed
        act, beta, lb = R._act()
        table = R.expert_table()
        n = flat.shape[0]
        x = flat if flat.dtype in (torch.float32, torch.bfloat16) else flat.to(torch.float32)
        x = T.contiguous_aligned(x)
        H, Lw, I, Is, E, k = R._H, self.latent, R._I, R._Is, R._E, R._k
        nbytes = int(_lib.lib().k3_moe_latent_layer_multi_workspace_size(n, H, Lw, I, Is, E, k))
        ws = _workspace.get(R.device, nbytes, "moe_latent_multi")
        out = torch.empty((n, H), dtype=out_dtype, device=R.device)
        _lib.call("k3_moe_latent_layer_decode_multi", T.ptr(x), T.dtype_code(x.dtype), T.ptr(R.gate_w),
                  T.ptr(R.gate_b), int(bool(c.moe_renormalize)), float(c.routed_scaling_factor), T.ptr(table),
                  T.ptr(self.down), T.ptr(self.up), T.ptr(self._norm32), float(c.rms_norm_eps), T.ptr(R.sh_gate),
                  T.ptr(R.sh_up), T.ptr(R.sh_down), T.ptr(out), T.dtype_code(out_dtype), n, H, Lw, I, Is, E, k,
                  ACTS[act], float(beta), float(lb or 0.0), T.ptr(ws), ws.numel(), T.stream(x))
        y = out.reshape(*orig[:-1], H)
        if not return_router:
            return y
        off = (ctypes.c_int64 * 5)()
        _lib.call("k3_moe_latent_layer_multi_workspace_offsets", n, H, Lw, I, Is, E, k, off)

        def rec(o, count, dt):
            return ws[o:o + 4 * count].view(dt).clone()

        r = RouterResult(rec(off[3], n * k, torch.int32).to(torch.int64).reshape(n, k),
                         rec(off[4], n * k, torch.float32).reshape(n, k),
                         rec(off[1], n * E, torch.float32).reshape(n, E),
                         rec(off[2], n * E, torch.float32).reshape(n, E))
        return y, r

    def grouped_forward(self, flat, return_router=False, out_dtype=torch.float32, orig=None):
        """Many tokens: route every token on x as given; h = x W_down^T on the BLAS library
        (bf16 for a bf16 x, fp32 for an fp32 x); the routed experts grouped by expert on the
        device (k3_moe_grouped_ffn); the norm in fp32; the up projection and the shared
        experts on the BLAS library with exact products and fp32 accumulation."""
        return self._forward_routed(flat, return_router, out_dtype, orig, moe_grouped_ffn)

    def multi_forward(self, flat, return_router=False, out_dtype=torch.float32, orig=None):
        """A few decode tokens (at most DECODE_TOKENS) with the dense projections on the BLAS
        library: as grouped_forward, with the routed experts run by moe_routed_decode, so
        every expert any token selects is read once against all the tokens routed to it.
        ``__call__`` runs the same step with every projection in HIP (_decode_multi)."""
        return self._forward_routed(flat, return_router, out_dtype, orig, moe_routed_decode)

    def _forward_routed(self, flat, return_router, out_dtype, orig, routed_fn):
        c = self.cfg
        orig = orig if orig is not None else flat.shape
        flat = flat.reshape(-1, flat.shape[-1])
        r = self.route(flat)
        h = _blas.mm_f32(flat, self.down)                                 # hidden -> latent
        if flat.dtype == torch.bfloat16:
            h = h.to(torch.bfloat16)                                      # the reference's bf16 matmul
        act, beta, lb = self._routed._act()
        y = routed_fn(h.contiguous(), r.expert_indices, r.expert_weights, self._routed.expert_table(),
                      int(c.moe_intermediate_size), act, beta, lb, out_dtype=torch.float32, validate=False)
        y = _rmsnorm32(y, self._norm32, float(c.rms_norm_eps))
        y = _blas.mm_f32(y, self.up)                                      # latent -> hidden
        if self._routed.sh_gate is not None:
            y = y + self.shared_forward(flat)
        y = y.to(out_dtype).reshape(*orig[:-1], orig[-1])
        return (y, r) if return_router else y


def moe_grouped_ffn(x: torch.Tensor, expert_indices: torch.Tensor, expert_weights: torch.Tensor,
                    table: torch.Tensor, intermediate: int, act: str = "silu", beta: float = 1.0,
                    linear_beta: float | None = None, out_dtype: torch.dtype = torch.float32,
                    validate: bool = True) -> torch.Tensor:
    """Routed experts for many tokens at once (prefill): x [T, H] bf16, expert_indices
    [T, k] (ids into the [E, 6] device pointer table), expert_weights [T, k] -> [T, H].

    The per-expert loop of LatentMoE.__call__ (moe.py:120-127) becomes a device grouping
    pass plus two grouped MFMA GEMMs and a fixed-order combine (k3_moe_grouped_ffn).
    ``validate`` checks the ids on the device first (one small device->host copy)."""
    if x.dim() != 2 or expert_indices.shape != expert_weights.shape or expert_indices.shape[0] != x.shape[0]:
        raise ValueError(f"x [T, H] with expert_indices/expert_weights [T, k] expected; got {tuple(x.shape)}, "
                         f"{tuple(expert_indices.shape)}, {tuple(expert_weights.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.to(torch.float32)
    T.require_device(x, expert_indices, expert_weights, table)
    n_tok, H = x.shape
    k = expert_indices.shape[1]
    E = table.shape[0]
    idx = expert_indices.to(torch.int32).contiguous()
    if validate and idx.numel():
        lo, hi = (int(v) for v in torch.stack([idx.min(), idx.max()]).tolist())
        if lo < 0 or hi >= E:
            raise ValueError(f"expert ids {lo}..{hi} outside 0..{E - 1}")
    w = expert_weights.to(torch.float32).contiguous()
    x = T.contiguous_aligned(x)
    out = torch.empty((n_tok, H), dtype=out_dtype, device=x.device)
    if n_tok == 0:
        return out
    nbytes = int(_lib.lib().k3_moe_grouped_workspace_size(n_tok, k, E, H, intermediate))
    ws = _workspace.get(x.device, nbytes, "moe_grouped")
    _lib.call("k3_moe_grouped_ffn", T.ptr(x), T.dtype_code(x.dtype), T.ptr(idx), T.ptr(w), T.ptr(table),
              T.ptr(out), T.dtype_code(out_dtype), n_tok, H, intermediate, E, k, _act_code(act), float(beta),
              float(linear_beta or 0.0), T.ptr(ws), ws.numel(), T.stream(x))
    return out


def moe_routed_decode(x: torch.Tensor, expert_indices: torch.Tensor, expert_weights: torch.Tensor,
                      table: torch.Tensor, intermediate: int, act: str = "silu", beta: float = 1.0,
                      linear_beta: float | None = None, out_dtype: torch.dtype = torch.float32,
                      validate: bool = True) -> torch.Tensor:
    """Routed experts for a few decode tokens: x [T, H] (T <= 8, bf16 or fp32),
    expert_indices / expert_weights [T, k] -> [T, H].  The per-expert loop of
    LatentMoE.__call__ (moe.py:119-127) as four launches (k3_moe_routed_decode): the union
    of the routed experts on the device, then every union expert's gate/up and down rows
    streamed once against all the tokens routed to it, then the fixed-order combine.  ``validate`` checks the ids on the
    device first (one small device->host copy); unchecked, out-of-range ids contribute
    nothing."""
    if x.dim() != 2 or expert_indices.shape != expert_weights.shape or expert_indices.shape[0] != x.shape[0]:
        raise ValueError(f"x [T, H] with expert_indices/expert_weights [T, k] expected; got {tuple(x.shape)}, "
                         f"{tuple(expert_indices.shape)}, {tuple(expert_weights.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float32):
        x = x.to(torch.float32)
    T.require_device(x, expert_indices, expert_weights, table)
    n_tok, H = x.shape
    k = expert_indices.shape[1]
    E = table.shape[0]
    idx = expert_indices.to(torch.int32).contiguous()
    if validate and idx.numel():
        lo, hi = (int(v) for v in torch.stack([idx.min(), idx.max()]).tolist())
        if lo < 0 or hi >= E:
            raise ValueError(f"expert ids {lo}..{hi} outside 0..{E - 1}")
    w = expert_weights.to(torch.float32).contiguous()
    x = T.contiguous_aligned(x)
    out = torch.empty((n_tok, H), dtype=out_dtype, device=x.device)
    if n_tok == 0:
        return out
    nbytes = int(_lib.lib().k3_moe_routed_workspace_size(n_tok, H, intermediate, E, k))
    ws = _workspace.get(x.device, nbytes, "moe_routed")
    _lib.call("k3_moe_routed_decode", T.ptr(x), T.dtype_code(x.dtype), T.ptr(idx), T.ptr(w), T.ptr(table),
              T.ptr(out), T.dtype_code(out_dtype), n_tok, H, intermediate, E, k, _act_code(act), float(beta),
              float(linear_beta or 0.0), T.ptr(ws), ws.numel(), T.stream(x))
    return out


def _act_torch(g, u, act, beta, lb):
    """Torch form of the activations for the unfused (debug) path only."""
    if act == "situ":
        a = beta * torch.tanh(g / beta) * torch.sigmoid(g)
        return a * (lb * torch.tanh(u / lb) if lb else u)
    return torch.nn.functional.silu(g) * u
