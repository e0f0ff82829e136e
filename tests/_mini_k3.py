"""A miniature Kimi-K3 for the integration gate: checkpoint writer, a HIP-backed decoder
stack and an fp64 oracle stack over the same tensors.

Restates the reference's synthetic-model gate (tests/test_synthetic_integration.py:104-184,
generator tools/make_synthetic_k3.py:87-110,132-252) at shapes the HIP kernels take:
three layers -- 0: KDA + dense MLP, 1: KDA + latent MoE, 2: MLA + latent MoE -- with the
real operations (sigmoid router with correction bias, SiTU, latent down/norm/up wrapper,
one shared expert, MXFP4 experts, NoPE MLA with the output gate, KDA with A_log padding).
The ranks are the kernels' fixed ones (MLA kv_lora_rank 512 and rope 64, KDA head_dim 128,
expert widths multiples of 128), not the reference's smaller mini shapes.

The decoder around the layers (token embedding, pre-norm residual blocks, final norm, tied
argmax head) is test scaffolding: it only has to be the same for every path it compares.
"""
from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import numpy as np

from oracle import kda as okda
from oracle import mla as omla
from oracle import moe as omoe
from oracle import mxfp4 as om

PROMPT = [7, 42, 128, 9]
NTOK = 6


@dataclass
class MiniCfg:
    hidden_size: int = 256
    vocab_size: int = 512
    num_hidden_layers: int = 3
    first_k_dense_replace: int = 1
    intermediate_size: int = 512
    rms_norm_eps: float = 1e-5
    # KDA (layers 0 and 1)
    kda_num_heads: int = 2
    kda_head_dim: int = 128
    kda_conv_size: int = 4
    kda_gate_lower_bound: float = -5.0
    # MLA (layer 2)
    num_attention_heads: int = 4
    q_lora_rank: int = 64
    kv_lora_rank: int = 512
    qk_nope_head_dim: int = 16
    qk_rope_head_dim: int = 64
    v_head_dim: int = 16
    mla_use_output_gate: bool = True
    # latent MoE (layers 1 and 2)
    num_experts: int = 8
    num_experts_per_token: int = 2
    num_shared_experts: int = 1
    moe_intermediate_size: int = 128
    routed_expert_hidden_size: int = 128
    routed_scaling_factor: float = 1.0
    moe_renormalize: bool = True
    situ_beta: float = 4.0
    situ_linear_beta: float = 25.0

    @property
    def q_head_dim(self) -> int:
        return self.qk_nope_head_dim + self.qk_rope_head_dim

    mla_layers = (2,)

    def is_mla(self, layer: int) -> bool:
        return layer in self.mla_layers

    def is_moe(self, layer: int) -> bool:
        return layer >= self.first_k_dense_replace


PFX = "language_model.model."


def layer_prefix(layer: int) -> str:
    return f"{PFX}layers.{layer}."


def build_checkpoint(out: Path, cfg: MiniCfg | None = None, seed: int = 0) -> dict:
    """Write the shards (one per layer plus one for the model tensors) with the checkpoint
    names the reference loader reads; return {name: (array as stored, dtype)}.  Dense
    tensors are bf16 (stored as their bit patterns), norms and KDA vectors fp32, experts
    MXFP4 from the oracle's encoder (E8M0 so the group max lands in [4, 8))."""
    from k3hip.checkpoint import write_safetensors

    cfg = cfg or MiniCfg()
    rng = np.random.default_rng(seed)
    H = cfg.hidden_size
    out = Path(out)
    out.mkdir(parents=True, exist_ok=True)
    allt = {}

    def bf(a):
        return om.bf16_bits(np.asarray(a, np.float32)), "BF16"

    def W(*shape, s=0.02):
        return (rng.standard_normal(shape) * s).astype(np.float32)

    for L in range(cfg.num_hidden_layers):
        t = {}
        p = layer_prefix(L)
        for n in ("input_layernorm", "post_attention_layernorm"):
            t[p + n + ".weight"] = bf(1.0 + W(H, s=0.01))
        attn = omla.random_mla_weights(rng, cfg) if cfg.is_mla(L) else okda.random_kda_weights(rng, cfg)
        for k, a in attn.items():
            if cfg.is_mla(L):
                t[p + "self_attn." + k] = bf(a)
            elif k.endswith("proj.weight"):
                t[p + "self_attn." + k] = bf(a)
            else:
                t[p + "self_attn." + k] = (np.ascontiguousarray(a, np.float32), "F32")
        if not cfg.is_moe(L):
            I = cfg.intermediate_size
            t[p + "mlp.gate_proj.weight"] = bf(W(I, H))
            t[p + "mlp.up_proj.weight"] = bf(W(I, H))
            t[p + "mlp.down_proj.weight"] = bf(W(H, I))
        else:
            m = p + "block_sparse_moe."
            Lw, I, Is = cfg.routed_expert_hidden_size, cfg.moe_intermediate_size, \
                cfg.moe_intermediate_size * cfg.num_shared_experts
            t[m + "gate.weight"] = bf(W(cfg.num_experts, H))
            t[m + "gate.e_score_correction_bias"] = (W(cfg.num_experts, s=0.1), "F32")
            t[m + "routed_expert_down_proj.weight"] = bf(W(Lw, H, s=0.05))
            t[m + "routed_expert_up_proj.weight"] = bf(W(H, Lw, s=0.05))
            t[m + "routed_expert_norm.weight"] = bf(1.0 + W(Lw, s=0.01))
            t[m + "shared_experts.gate_proj.weight"] = bf(W(Is, H))
            t[m + "shared_experts.up_proj.weight"] = bf(W(Is, H))
            t[m + "shared_experts.down_proj.weight"] = bf(W(H, Is))
            for e in range(cfg.num_experts):
                for w, shape in (("w1", (I, Lw)), ("w3", (I, Lw)), ("w2", (Lw, I))):
                    pk, sc = om.encode_mxfp4(W(*shape, s=0.05))
                    t[f"{m}experts.{e}.{w}.weight_packed"] = (pk, "U8")
                    t[f"{m}experts.{e}.{w}.weight_scale"] = (sc, "U8")
        write_safetensors(out / f"model-{L + 1:05d}-of-{cfg.num_hidden_layers + 1:05d}.safetensors", t)
        allt.update(t)
    t = {PFX + "embed_tokens.weight": bf(W(cfg.vocab_size, H, s=0.05)),
         "language_model.lm_head.weight": bf(W(cfg.vocab_size, H, s=0.05)),
         PFX + "norm.weight": bf(1.0 + W(H, s=0.01))}
    write_safetensors(out / f"model-{cfg.num_hidden_layers + 1:05d}-of-{cfg.num_hidden_layers + 1:05d}.safetensors", t)
    allt.update(t)
    return allt


def _value(arr, dtype):
    return om.bf16_from_bits(arr).astype(np.float64) if dtype == "BF16" else np.asarray(arr, np.float64)


class OracleModel:
    """The decoder in float64 on the oracle's layers: every call recomputes the whole
    sequence (KDA from a zero state, MLA with the causal mask)."""

    def __init__(self, tensors: dict, cfg: MiniCfg | None = None):
        self.cfg = cfg or MiniCfg()
        self.t = tensors

    def _v(self, name):
        return _value(*self.t[name])

    def _attn_w(self, L):
        p = layer_prefix(L) + "self_attn."
        return {n[len(p):]: self._v(n) for n in self.t if n.startswith(p)}

    def _moe(self, L, h):
        c, p = self.cfg, layer_prefix(L) + "block_sparse_moe."
        experts = [tuple((self.t[f"{p}experts.{e}.{w}.weight_packed"][0], self.t[f"{p}experts.{e}.{w}.weight_scale"][0])
                         for w in ("w1", "w3", "w2")) for e in range(c.num_experts)]
        shared = tuple(self._v(p + f"shared_experts.{n}_proj.weight") for n in ("gate", "up", "down"))
        y, idx, _ = omoe.latent_moe(h, self._v(p + "gate.weight"), self._v(p + "gate.e_score_correction_bias"),
                                    self._v(p + "routed_expert_down_proj.weight"),
                                    self._v(p + "routed_expert_up_proj.weight"),
                                    self._v(p + "routed_expert_norm.weight"), experts, shared,
                                    c.num_experts_per_token, c.moe_renormalize, c.routed_scaling_factor,
                                    c.situ_beta, c.situ_linear_beta, c.rms_norm_eps, "situ")
        return y

    def logits(self, ids: list[int]) -> np.ndarray:
        c = self.cfg
        x = self._v(PFX + "embed_tokens.weight")[ids][None]          # [1, T, H]
        for L in range(c.num_hidden_layers):
            p = layer_prefix(L)
            h = omoe.rmsnorm(x, self._v(p + "input_layernorm.weight"), c.rms_norm_eps)
            if c.is_mla(L):
                o = omla.mla_layer_expanded(c, self._attn_w(L), h)
            else:
                o = okda.kda_layer(c, self._attn_w(L), h)[0]
            x = x + o
            h = omoe.rmsnorm(x, self._v(p + "post_attention_layernorm.weight"), c.rms_norm_eps)[0]
            if c.is_moe(L):
                m = self._moe(L, h)
            else:
                m = omoe.dense_ffn(h, self._v(p + "mlp.gate_proj.weight"), self._v(p + "mlp.up_proj.weight"),
                                   self._v(p + "mlp.down_proj.weight"), kind="situ", beta=c.situ_beta,
                                   linear_beta=c.situ_linear_beta)[0]
            x = x + m[None]
        x = omoe.rmsnorm(x, self._v(PFX + "norm.weight"), c.rms_norm_eps)
        return x[0, -1] @ self._v("language_model.lm_head.weight").T

    def generate(self, prompt: list[int], n: int) -> list[int]:
        ids, out = list(prompt), []
        for _ in range(n):
            tok = int(np.argmax(self.logits(ids)))
            out.append(tok)
            ids.append(tok)
        return out


class GpuModel:
    """The same decoder on the HIP layers, incremental: a KDA state and convolution window
    per KDA layer and an MLA cache, so every generated token is one decode step.  The
    residual stream is fp32 (the layers' validation-precision input).  ``fused`` picks the
    MoE path (fused kernels, or the reference loop with unfused projections); ``resident``
    keeps every expert of a layer in one device allocation instead of reading each
    projection from the checkpoint when it is used."""

    def __init__(self, src, cfg: MiniCfg | None = None, fused: bool = True, resident: bool = False):
        import torch
        from k3hip.kda import KDAAttention
        from k3hip.mla import MLAAttention
        from k3hip.moe import LatentMoE

        self.torch = torch
        self.cfg = c = cfg or MiniCfg()
        self.src = src
        f32 = lambda n: src.tensor(n, torch.float32)  # noqa: E731
        self.embed = f32(PFX + "embed_tokens.weight")
        self.head = f32("language_model.lm_head.weight")
        self.norm = f32(PFX + "norm.weight")
        self.layers = []
        for L in range(c.num_hidden_layers):
            p = layer_prefix(L)
            keys = MLAAttention.KEYS if c.is_mla(L) else KDAAttention.KEYS
            w = {k: src.tensor(p + "self_attn." + k) for k in keys}
            attn = MLAAttention(c, w) if c.is_mla(L) else KDAAttention(c, w)
            if c.is_moe(L):
                esrc = src.load_experts(L, c.num_experts).source if resident else src.expert_source
                mlp = LatentMoE(c, L, src.moe_weights(L), esrc, fused=fused)
            else:
                mlp = tuple(f32(p + f"mlp.{n}_proj.weight") for n in ("gate", "up", "down"))
            self.layers.append((f32(p + "input_layernorm.weight"), attn, f32(p + "post_attention_layernorm.weight"),
                                mlp))
        self.reset()

    def reset(self):
        self.kda = {}
        self.cache = None

    def _rms(self, x, w):
        t = self.torch
        return x * t.rsqrt((x * x).mean(-1, keepdim=True) + self.cfg.rms_norm_eps) * w

    def _dense_mlp(self, h, w):
        from k3hip.moe import _act_torch
        g, u = h @ w[0].T, h @ w[1].T
        return _act_torch(g, u, "situ", self.cfg.situ_beta, self.cfg.situ_linear_beta) @ w[2].T

    def forward(self, ids: list[int]):
        """Feed the new tokens; returns the logits of the last one (fp32)."""
        t, c = self.torch, self.cfg
        x = self.embed[t.tensor(ids, device=self.embed.device)][None]   # [1, Tn, H]
        for L, (n_in, attn, n_post, mlp) in enumerate(self.layers):
            h = self._rms(x, n_in)
            if c.is_mla(L):
                o, self.cache = attn(h, self.cache)
            else:
                st, conv = self.kda.get(L, (None, None))
                o, st, conv = attn(h, st, conv)
                self.kda[L] = (st, conv)
            x = x + o
            h = self._rms(x, n_post)
            m = mlp(h) if c.is_moe(L) else self._dense_mlp(h, mlp)
            x = x + m
        x = self._rms(x, self.norm)
        return x[0, -1] @ self.head.T

    def generate(self, prompt: list[int], n: int) -> list[int]:
        self.reset()
        out, nxt = [], list(prompt)
        for _ in range(n):
            tok = int(self.torch.argmax(self.forward(nxt)))
            out.append(tok)
            nxt = [tok]
        return out
