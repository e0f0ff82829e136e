"""Latent-MLA absorbed decode on MI355X -- the counterpart of
air_llm/models/kimi_k3/attention_mla.py (``MLACache``, ``MLAAttention``).

``mla_decode_absorbed(q_nope, q_rot, wk, wv, lat, rot, scale)`` is the attention core of
``MLAAttention.__call__`` for one decode token (``attention_mla.py:193-212``): it runs on
the latent cache in place, bf16 or the reference's fp32 (four HIP launches: query
absorption, split-T flash decoding on bf16 MFMA with hi/lo-split fp32 operands -- fp32
cache rows split into hi/lo bf16 planes as they are staged --, log-sum-exp merge of the
splits, the W_UV absorption) and returns ``[H, v_head_dim]``.

``MLACache`` keeps the reference's surface (``latent``/``rot`` backing buffers with spare
capacity, valid prefix ``length``, ``append`` with chunked doubling growth, ``view``,
``bytes_per_token``, ``nbytes_used``, ``attention_mla.py:62-117``), with bf16 device storage
by default: the kernel reads the valid prefix directly, so ``view`` does not upcast.

``MLAAttention(cfg, w)`` keeps the reference constructor and ``__call__(x, cache)``.  With
bf16 projection weights (the checkpoint dtype) the decode step (one token, batch 1) is
``k3_mla_step_decode``: the projections, RMSNorms, cache append, attention core, output
gate and o_proj in seven HIP launches.  With other weight dtypes the projections are torch
fp32 matmuls around the HIP core.  Prefill (T > 1) keeps the reference's dense masked form
in torch on the GPU.

The cache defaults to bf16 (``cfg.mla_cache_dtype``), which the HIP core reads in place; the
reference's default is an fp32 cache (``attention_mla.py:164``), which it calls lossless.
An fp32 cache (``mla_cache_dtype=torch.float32``, or a caller's fp32 ``MLACache``) is
accepted: a decode token on it runs the HIP core on the fp32 rows
(``k3_mla_decode_absorbed_f32``; with bf16 ``kv_b``, the checkpoint dtype, whose halves the
core takes as they are), the projections around it in fp32; fp32 ``kv_b`` (validation mode)
and prefill run the fp32 masked form.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib, _workspace
from . import _torch as T

CACHE_STEP = 256
KV_LORA_RANK = 512
ROPE_DIM = 64


def _round_up(n: int, step: int) -> int:
    return ((n + step - 1) // step) * step


@dataclass
class MLACache:
    """Latent KV cache (attention_mla.py:62-117): ``latent`` [B, cap, kv_lora_rank] and
    ``rot`` [B, cap, rope] backing buffers; the first ``length`` positions are valid."""
    latent: torch.Tensor
    rot: torch.Tensor
    length: int = 0

    @property
    def capacity(self) -> int:
        return self.latent.shape[1]

    def view(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The valid prefix, in the storage dtype (the kernels read bf16 directly)."""
        return self.latent[:, :self.length], self.rot[:, :self.length]

    def reserve(self, n: int) -> "MLACache":
        """Capacity for n more positions, growing by doubling (floor CACHE_STEP) when full
        (attention_mla.py:93-101)."""
        need = self.length + n
        if need > self.capacity:
            cap = _round_up(max(need, 2 * self.capacity, CACHE_STEP), CACHE_STEP)
            self.latent = _grown(self.latent, cap, self.length)
            self.rot = _grown(self.rot, cap, self.length)
        return self

    def append(self, c_new: torch.Tensor, r_new: torch.Tensor) -> "MLACache":
        """Write T new positions, growing by doubling (floor CACHE_STEP) when full."""
        n = c_new.shape[1]
        need = self.length + n
        self.reserve(n)
        self.latent[:, self.length:need] = c_new.to(self.latent.dtype)
        self.rot[:, self.length:need] = r_new.to(self.rot.dtype)
        self.length = need
        return self

    def bytes_per_token(self) -> float:
        return (self.latent.shape[2] * self.latent.element_size()
                + self.rot.shape[2] * self.rot.element_size())

    def nbytes_used(self) -> int:
        """Bytes of the valid prefix (what the cache would cost if trimmed)."""
        return int(self.rot.shape[0] * self.length * self.bytes_per_token())


def _grown(buf: torch.Tensor, cap: int, keep: int) -> torch.Tensor:
    out = torch.zeros((buf.shape[0], cap, buf.shape[2]), dtype=buf.dtype, device=buf.device)
    if keep:
        out[:, :keep] = buf[:, :keep]
    return out


def new_cache(B: int, kv_lora_rank: int, rope: int, T: int, dtype=torch.bfloat16,
              device="cuda") -> MLACache:
    """``_new_cache`` (attention_mla.py:127-134) without the quantised option."""
    cap = _round_up(max(T, CACHE_STEP), CACHE_STEP)
    return MLACache(torch.zeros((B, cap, kv_lora_rank), dtype=dtype, device=device),
                    torch.zeros((B, cap, rope), dtype=dtype, device=device), 0)


def _heads(w: torch.Tensor, name: str) -> torch.Tensor:
    """[1, H, a, r] or [H, a, r] bf16 -> contiguous [H, a, r]."""
    if w.dim() == 4:
        if w.shape[0] != 1:
            raise ValueError(f"{name} must be [1, H, d, r] or [H, d, r]; got {tuple(w.shape)}")
        w = w[0]
    if w.dim() != 3:
        raise ValueError(f"{name} must be [1, H, d, r] or [H, d, r]; got {tuple(w.shape)}")
    if w.dtype != torch.bfloat16:
        raise TypeError(f"{name} must be bfloat16 (the checkpoint dtype)")
    return T.contiguous_aligned(w)


def _cache_rows(c: torch.Tensor, width: int, name: str) -> torch.Tensor:
    """[T, width] or [1, T, width] bf16 or fp32 with unit inner stride and a row stride of
    whole 16-byte units (cache backing buffers qualify); copies otherwise."""
    if c.dim() == 3:
        if c.shape[0] != 1:
            raise ValueError(f"{name}: the decode kernel takes batch 1; got {tuple(c.shape)}")
        c = c[0]
    if c.dim() != 2 or c.shape[1] != width:
        raise ValueError(f"{name} must be [T, {width}]; got {tuple(c.shape)}")
    if c.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"{name} must be bfloat16 or float32 (the latent cache dtypes); got {c.dtype}")
    if c.stride(1) != 1 or c.stride(0) % (16 // c.element_size()) or c.data_ptr() % 16:
        c = c.contiguous()
        if c.data_ptr() % 16:
            c = c.clone()
    return c


def mla_decode_absorbed(q_nope: torch.Tensor, q_rot: torch.Tensor, wk: torch.Tensor, wv: torch.Tensor,
                        lat: torch.Tensor, rot: torch.Tensor, scale: float,
                        out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Absorbed MLA attention for one query per head (attention_mla.py:193-212, T == 1).

    q_nope [H, nope], q_rot [H, rope] (bf16 or fp32); wk [H, nope, r], wv [H, v, r]
    (bf16, or the reference's [1, H, ., r] views); lat [T, r], rot [T, rope] cache rows (or
    [1, T, .]), both bf16 (k3_mla_decode_absorbed) or both fp32, the reference's default
    cache dtype (k3_mla_decode_absorbed_f32).  Returns o [H, v] in out_dtype (fp32
    accumulation throughout).
    """
    if q_nope.dim() != 2 or q_rot.dim() != 2 or q_nope.shape[0] != q_rot.shape[0]:
        raise ValueError(f"q_nope [H, nope] and q_rot [H, rope] expected; got {tuple(q_nope.shape)}, "
                         f"{tuple(q_rot.shape)}")
    H, nope = q_nope.shape
    wk = _heads(wk, "wk")
    wv = _heads(wv, "wv")
    r = wk.shape[2]
    if tuple(wk.shape) != (H, nope, r) or wv.shape[0] != H or wv.shape[2] != r:
        raise ValueError(f"weight shapes {tuple(wk.shape)}, {tuple(wv.shape)} do not match q [{H}, {nope}]")
    lat = _cache_rows(lat, r, "lat")
    rot = _cache_rows(rot, q_rot.shape[1], "rot")
    if lat.shape[0] != rot.shape[0]:
        raise ValueError(f"lat has {lat.shape[0]} tokens, rot {rot.shape[0]}")
    if lat.dtype != rot.dtype:
        raise TypeError(f"lat and rot must share one dtype; got {lat.dtype}, {rot.dtype}")
    T.require_device(q_nope, q_rot, wk, wv, lat, rot)
    qdt = torch.bfloat16 if (q_nope.dtype == torch.bfloat16 and q_rot.dtype == torch.bfloat16) else torch.float32
    q_nope = q_nope.to(qdt)
    q_rot = q_rot.to(qdt)
    if q_nope.stride(1) != 1:
        q_nope = q_nope.contiguous()
    if q_rot.stride(1) != 1:
        q_rot = q_rot.contiguous()
    V = wv.shape[1]
    out = torch.empty((H, V), dtype=out_dtype, device=lat.device)
    ntok = lat.shape[0]
    ws_bytes = int(_lib.lib().k3_mla_workspace_size(H, ntok))
    ws = _workspace.get(lat.device, ws_bytes, "mla")
    entry = "k3_mla_decode_absorbed" if lat.dtype == torch.bfloat16 else "k3_mla_decode_absorbed_f32"
    _lib.call(entry, T.ptr(q_nope), T.ptr(q_rot), q_nope.stride(0), q_rot.stride(0),
              T.dtype_code(qdt),
              T.ptr(wk), T.ptr(wv), T.ptr(lat), lat.stride(0), T.ptr(rot), rot.stride(0), ntok, H, r,
              q_rot.shape[1], nope, V, float(scale), T.ptr(out), T.dtype_code(out_dtype), out.stride(0),
              T.ptr(ws), ws.numel(), T.stream(lat))
    return out


def _rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """KimiRMSNorm in fp32 (ops.py:11-14)."""
    xf = x.to(torch.float32)
    return w.to(torch.float32) * (xf * torch.rsqrt((xf * xf).mean(-1, keepdim=True) + eps))


class MLAAttention:
    """Drop-in for MLAAttention (attention_mla.py:137-216).  Weights are the checkpoint
    tensors as-is ([out, in], applied as x @ W.T), on the GPU."""

    KEYS = ("q_a_proj.weight", "q_a_layernorm.weight", "q_b_proj.weight",
            "kv_a_proj_with_mqa.weight", "kv_a_layernorm.weight", "kv_b_proj.weight",
            "g_proj.weight", "o_proj.weight")

    def __init__(self, cfg, w: dict):
        self.cfg = cfg
        self.q_a, self.q_an, self.q_b = w["q_a_proj.weight"], w["q_a_layernorm.weight"], w["q_b_proj.weight"]
        self.kv_a, self.kv_an = w["kv_a_proj_with_mqa.weight"], w["kv_a_layernorm.weight"]
        self.kv_b = w["kv_b_proj.weight"]
        self.g_w, self.o_w = w.get("g_proj.weight"), w["o_proj.weight"]
        nh, nope = cfg.num_attention_heads, cfg.qk_nope_head_dim
        kb = self.kv_b.to(torch.bfloat16).reshape(nh, nope + cfg.v_head_dim, cfg.kv_lora_rank)
        self.wk = kb[:, :nope, :].contiguous()        # [H, nope, r], bf16 for the HIP core
        self.wv = kb[:, nope:, :].contiguous()        # [H, v, r]
        kb32 = self.kv_b.to(torch.float32).reshape(nh, nope + cfg.v_head_dim, cfg.kv_lora_rank)
        self._wk32, self._wv32 = kb32[:, :nope, :], kb32[:, nope:, :]   # the fp32 form uses kv_b as given
        self.cache_dtype = getattr(cfg, "mla_cache_dtype", torch.bfloat16)
        mats = [self.q_a, self.q_b, self.kv_a, self.o_w] + ([self.g_w] if self.g_w is not None else [])
        self.fused_step = (all(m.dtype == torch.bfloat16 and m.is_cuda for m in mats)
                           and self.cache_dtype == torch.bfloat16
                           and cfg.kv_lora_rank == KV_LORA_RANK and cfg.qk_rope_head_dim == ROPE_DIM)
        if self.fused_step:
            self._mats = {k: T.contiguous_aligned(m) for k, m in
                          (("q_a", self.q_a), ("q_b", self.q_b), ("kv_a", self.kv_a), ("o", self.o_w))}
            self._mats["g"] = T.contiguous_aligned(self.g_w) if self.g_w is not None else None
            self._q_an32 = T.contiguous_aligned(self.q_an.to(torch.float32))
            self._kv_an32 = T.contiguous_aligned(self.kv_an.to(torch.float32))

    @staticmethod
    def _mm(a: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        """a @ w^T with fp32 output.  bf16 a against bf16 w runs as one BLAS GEMM with fp32
        accumulation and output (the same products as in fp32, no weight copy); otherwise
        both operands go to fp32."""
        if a.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and a.is_cuda:
            try:
                return torch.mm(a.reshape(-1, a.shape[-1]), w.t(), out_dtype=torch.float32).reshape(
                    *a.shape[:-1], w.shape[0])
            except (RuntimeError, TypeError):
                pass
        return a.to(torch.float32) @ w.to(torch.float32).T

    def __call__(self, x: torch.Tensor, cache: MLACache | None = None):
        c = self.cfg
        B, Tn, _ = x.shape
        if self.fused_step and B == 1 and Tn == 1 and (cache is None or cache.latent.dtype == torch.bfloat16):
            return self.decode_step(x, cache)
        nh, qhd, vhd = c.num_attention_heads, c.q_head_dim, c.v_head_dim
        nope, rope, klr = c.qk_nope_head_dim, c.qk_rope_head_dim, c.kv_lora_rank
        eps = c.rms_norm_eps
        q = self._mm(_rmsnorm(self._mm(x, self.q_a), self.q_an, eps), self.q_b)
        q = q.reshape(B, Tn, nh, qhd).transpose(1, 2)               # [B, H, T, qhd]
        ckv = self._mm(x, self.kv_a)
        c_new = _rmsnorm(ckv[..., :klr], self.kv_an, eps)
        r_new = ckv[..., klr:]
        if cache is None:
            cache = new_cache(B, klr, rope, Tn, self.cache_dtype, x.device)
        cache.append(c_new, r_new)
        lat, rot = cache.view()
        scale = qhd ** -0.5
        # one query token: the HIP core, over a bf16 cache or the reference's default fp32
        # cache; an fp32 cache with fp32 kv_b (validation mode) keeps the exact fp32 form,
        # since the core takes W_UK / W_UV in bf16
        if Tn == 1 and B == 1 and (lat.dtype == torch.bfloat16 or
                                   (lat.dtype == torch.float32 and self.kv_b.dtype == torch.bfloat16)):
            o = mla_decode_absorbed(q[0, :, 0, :nope], q[0, :, 0, nope:], self.wk, self.wv,
                                    lat[0], rot[0], scale).reshape(1, 1, nh * vhd)
        else:
            o = self._dense(q, lat, rot, scale).transpose(1, 2).reshape(B, Tn, nh * vhd)
        if getattr(c, "mla_use_output_gate", False):
            o = o * torch.sigmoid(self._mm(x, self.g_w))
        return self._mm(o, self.o_w), cache

    def decode_step(self, x: torch.Tensor, cache: MLACache | None = None):
        """One token at batch 1 through k3_mla_step_decode (attention_mla.py:168-216): the
        new latent row is written into the cache at position ``cache.length``."""
        c = self.cfg
        nh, nope, rope, vhd, klr = (c.num_attention_heads, c.qk_nope_head_dim, c.qk_rope_head_dim,
                                    c.v_head_dim, c.kv_lora_rank)
        hidden, ql = x.shape[-1], self.q_a.shape[0]
        if cache is None:
            cache = new_cache(1, klr, rope, 1, self.cache_dtype, x.device)
        cache.reserve(1)
        pos = cache.length
        xin = T.contiguous_aligned(x.reshape(hidden))
        if xin.dtype not in (torch.float32, torch.bfloat16):
            xin = xin.to(torch.float32)
        lat, rot = cache.latent[0], cache.rot[0]
        nbytes = int(_lib.lib().k3_mla_step_workspace_size(hidden, ql, nh, nope, rope, vhd, klr, pos + 1))
        ws = _workspace.get(x.device, nbytes, "mla_step")
        out = torch.empty(hidden, dtype=torch.float32, device=x.device)
        m = self._mats
        _lib.call("k3_mla_step_decode", T.ptr(xin), T.dtype_code(xin.dtype), T.ptr(m["q_a"]), T.ptr(self._q_an32),
                  T.ptr(m["q_b"]), T.ptr(m["kv_a"]), T.ptr(self._kv_an32), T.ptr(self.wk), T.ptr(self.wv),
                  T.ptr(m["g"] if getattr(c, "mla_use_output_gate", False) else None), T.ptr(m["o"]), T.ptr(lat),
                  lat.stride(0), T.ptr(rot), rot.stride(0), cache.capacity, pos, float(c.rms_norm_eps),
                  float(c.q_head_dim ** -0.5), T.ptr(out), _lib.K3_F32, hidden, ql, nh, nope, rope, vhd, klr,
                  T.ptr(ws), ws.numel(), T.stream(xin))
        cache.length = pos + 1
        return out.reshape(1, 1, hidden), cache

    # bytes of fp32 scores one query chunk of the multi-token form may hold (the scores and
    # probabilities of a 2048-token prompt over a 32768-token cache at 64 heads would be 17 GB
    # each if formed at once)
    DENSE_SCORE_BYTES = 1 << 28

    def _dense(self, q, lat, rot, scale):
        """Multi-token form (prefill): absorbed scores with the causal mask, fp32, in query
        chunks whose scores stay within DENSE_SCORE_BYTES (every query row's softmax is its
        own, so the chunks are independent)."""
        nope = self.cfg.qk_nope_head_dim
        latf, rotf = lat.to(torch.float32), rot.to(torch.float32)
        latT = latf.unsqueeze(1).transpose(-1, -2).contiguous()      # [B, 1, r, Tk]
        rotT = rotf.unsqueeze(1).transpose(-1, -2).contiguous()
        wvT = self._wv32.transpose(-1, -2).contiguous()
        B, H, Tq = q.shape[0], q.shape[1], q.shape[2]
        Tk = latf.shape[1]
        chunk = max(1, min(Tq, self.DENSE_SCORE_BYTES // max(1, B * H * Tk * 4)))
        ki = torch.arange(Tk, device=q.device).reshape(1, -1)
        outs = []
        for t0 in range(0, Tq, chunk):
            qc = q[:, :, t0:t0 + chunk]
            qa = qc[..., :nope] @ self._wk32                          # [B, H, t, r]
            s = (qa @ latT + qc[..., nope:] @ rotT) * scale
            qi = torch.arange(Tk - Tq + t0, Tk - Tq + t0 + qc.shape[2], device=q.device).reshape(-1, 1)
            s = s.masked_fill(ki > qi, float("-inf"))
            p = torch.softmax(s, dim=-1)
            outs.append((p @ latf.unsqueeze(1)) @ wvT)
        return outs[0] if len(outs) == 1 else torch.cat(outs, dim=2)
