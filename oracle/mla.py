"""Latent-MLA decode oracle (test infrastructure only).

Restates the absorbed attention core of ``air_llm/models/kimi_k3/attention_mla.py:193-212``
for one decode query per head (T == 1, so no causal mask, ``attention_mla.py:200-207``):

    qa[h]     = q_nope[h] @ W_UK[h]                    # [r]   (W_UK[h] is [nope, r])
    s[h, t]   = (qa[h] . lat[t] + q_rot[h] . rot[t]) * scale
    p[h, :]   = softmax(s[h, :])                        # fp32 softmax in the reference
    ctx[h]    = sum_t p[h, t] * lat[t]                  # [r]
    out[h]    = W_UV[h] @ ctx[h]                        # [v]   (W_UV[h] is [v, r])

and the expanded form it is algebraically equal to (``k3ref/layers.py:152-185``,
``tests/test_mla_cache.py:136-171``): per-head keys ``[W_UK[h] @ lat[t], rot[t]]`` and
values ``W_UV[h] @ lat[t]``.  Both in float64.

Pinning (``tests/test_oracle_mla.py``): absorbed == expanded (the reference's gate N3,
``tests/test_mla_cache.py:258-274``) on random inputs; a single cached token returns
``W_UV @ lat[0]`` exactly (softmax of one score is 1); identical cached tokens return the
same; a constant score shift leaves the output unchanged; the split-T log-sum-exp merge
(the flash-decoding combine) equals the one-shot softmax.
"""
from __future__ import annotations

import numpy as np


def mla_decode_absorbed(q_nope, q_rot, w_uk, w_uv, lat, rot, scale):
    """q_nope [H, nope], q_rot [H, rope], w_uk [H, nope, r], w_uv [H, v, r],
    lat [T, r], rot [T, rope] -> out [H, v] (float64).  Also returns (qa, probs, ctx)."""
    f = lambda a: np.asarray(a, dtype=np.float64)  # noqa: E731
    q_nope, q_rot, w_uk, w_uv, lat, rot = map(f, (q_nope, q_rot, w_uk, w_uv, lat, rot))
    qa = np.einsum("hn,hnr->hr", q_nope, w_uk)
    s = (qa @ lat.T + q_rot @ rot.T) * scale
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    p = e / e.sum(axis=-1, keepdims=True)
    ctx = p @ lat
    out = np.einsum("hvr,hr->hv", w_uv, ctx)
    return out, qa, p, ctx


def mla_decode_expanded(q_nope, q_rot, w_uk, w_uv, lat, rot, scale):
    """Same attention through materialised per-head keys/values."""
    f = lambda a: np.asarray(a, dtype=np.float64)  # noqa: E731
    q_nope, q_rot, w_uk, w_uv, lat, rot = map(f, (q_nope, q_rot, w_uk, w_uv, lat, rot))
    H = q_nope.shape[0]
    out = np.empty((H, w_uv.shape[1]))
    for h in range(H):
        k_pass = lat @ w_uk[h].T                     # [T, nope]
        v = lat @ w_uv[h].T                          # [T, v]
        key = np.concatenate([k_pass, rot], axis=1)  # [T, nope + rope]
        q = np.concatenate([q_nope[h], q_rot[h]])
        s = key @ q * scale
        s -= s.max()
        p = np.exp(s)
        p /= p.sum()
        out[h] = p @ v
    return out


def split_merge_softmax(scores: np.ndarray, values: np.ndarray, splits: int):
    """Flash-decoding combine in float64: softmax-weighted sum of ``values`` computed per
    T-split with (max, sum) partials and a log-sum-exp merge.  scores [T], values [T, d]."""
    scores = np.asarray(scores, np.float64)
    values = np.asarray(values, np.float64)
    parts = []
    for blk in np.array_split(np.arange(scores.shape[0]), splits):
        m = scores[blk].max()
        w = np.exp(scores[blk] - m)
        parts.append((m, w.sum(), w @ values[blk]))
    gm = max(m for m, _, _ in parts)
    den = sum(l * np.exp(m - gm) for m, l, _ in parts)
    num = sum(a * np.exp(m - gm) for m, _, a in parts)
    return num / den


def _rmsnorm64(x, w, eps):
    return w * (x / np.sqrt((x * x).mean(-1, keepdims=True) + eps))


def mla_layer_expanded(cfg, w: dict, x: np.ndarray) -> np.ndarray:
    """Whole MLA layer for a full sequence in float64, expanded form with the causal
    mask: the structure of the reference's independent oracle
    (``tests/test_mla_cache.py:136-171``; layer semantics ``k3ref/layers.py:152-185``).

    ``w`` holds the checkpoint tensors named in ``attention_mla.py:139-141``; ``x`` is
    [B, T, hidden].  The queries sit at positions 0..T-1, each sees positions <= its own.
    """
    x = np.asarray(x, np.float64)
    B, T, _ = x.shape
    nh, nope, rope = cfg.num_attention_heads, cfg.qk_nope_head_dim, cfg.qk_rope_head_dim
    vhd, klr, eps = cfg.v_head_dim, cfg.kv_lora_rank, cfg.rms_norm_eps
    qhd = nope + rope
    f = {k: np.asarray(v, np.float64) for k, v in w.items()}
    q = _rmsnorm64(x @ f["q_a_proj.weight"].T, f["q_a_layernorm.weight"], eps) @ f["q_b_proj.weight"].T
    q = q.reshape(B, T, nh, qhd).transpose(0, 2, 1, 3)
    ckv = x @ f["kv_a_proj_with_mqa.weight"].T
    kv = _rmsnorm64(ckv[..., :klr], f["kv_a_layernorm.weight"], eps) @ f["kv_b_proj.weight"].T
    kv = kv.reshape(B, T, nh, nope + vhd).transpose(0, 2, 1, 3)
    k_rot = np.broadcast_to(ckv[..., klr:].reshape(B, 1, T, rope), (B, nh, T, rope))
    key = np.concatenate([kv[..., :nope], k_rot], axis=-1)
    s = q @ key.transpose(0, 1, 3, 2) * qhd ** -0.5
    s = s + np.where(np.arange(T)[None, :] > np.arange(T)[:, None], -np.inf, 0.0)
    s -= s.max(-1, keepdims=True)
    e = np.exp(s)
    p = e / e.sum(-1, keepdims=True)
    o = (p @ kv[..., nope:]).transpose(0, 2, 1, 3).reshape(B, T, nh * vhd)
    if getattr(cfg, "mla_use_output_gate", False):
        o = o / (1.0 + np.exp(-(x @ f["g_proj.weight"].T)))
    return o @ f["o_proj.weight"].T


def random_mla_weights(rng, cfg, scale: float = 0.5) -> dict:
    """Random float32 checkpoint tensors at cfg's shapes (the reference test's recipe:
    N(0,1)/sqrt(fan_in) * scale, RMSNorm gains near 1, ``tests/test_mla_cache.py:77-94``)."""
    nh, nope, rope = cfg.num_attention_heads, cfg.qk_nope_head_dim, cfg.qk_rope_head_dim
    hid, ql, klr, vhd = cfg.hidden_size, cfg.q_lora_rank, cfg.kv_lora_rank, cfg.v_head_dim

    def lin(o, i):
        return (rng.standard_normal((o, i)) / np.sqrt(i) * scale).astype(np.float32)

    return {
        "q_a_proj.weight": lin(ql, hid),
        "q_a_layernorm.weight": (1.0 + 0.1 * rng.standard_normal(ql)).astype(np.float32),
        "q_b_proj.weight": lin(nh * (nope + rope), ql),
        "kv_a_proj_with_mqa.weight": lin(klr + rope, hid),
        "kv_a_layernorm.weight": (1.0 + 0.1 * rng.standard_normal(klr)).astype(np.float32),
        "kv_b_proj.weight": lin(nh * (nope + vhd), klr),
        "g_proj.weight": lin(nh * vhd, hid),
        "o_proj.weight": lin(hid, nh * vhd),
    }
