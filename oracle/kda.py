"""Kimi Delta Attention recurrence oracle (test infrastructure only).

Restates ``KDAAttention._recurrent`` (``air_llm/models/kimi_k3/attention_kda.py:65-90``),
which follows the vendored upstream ``naive_recurrent_kda``
(``k3ref/_vendor/kda_naive.py:46-60``), in float64.  For every step i and value head h,
with the state S [K, V]:

    S   = S * exp(g_i[h])[:, None]                  # per-key-channel decay (log space)
    S   = S + (beta_i[h] * k_i[h]) (x) (v_i[h] - k_i[h] . S)      # delta rule
    o_i = (scale * q_i[h]) . S                      # read-out after the update

q and k may have fewer heads than v (``HV`` a multiple of ``H``; value head h reads q/k
head ``h // (HV // H)``, the repeat_interleave of kda_naive.py:49-50).  K3's layers use
H == HV == 96, K == V == 128, scale = K**-0.5.

Pinning (``tests/test_oracle_kda.py``): scalar triple loops on tiny shapes; the delta
rule's defining property (with beta = 1 and a unit key, ``k . S_new == v`` whatever S and
the decay were); a zero state (``S_1 = beta k (x) v``, ``o = scale beta (q.k) v``); beta = 0
(pure decay, ``o = scale q . (S exp(g))``); step-by-step equals one multi-step call; and
planted mistakes (the delta taken on the undecayed state, the read-out before the update)
are caught.
"""
from __future__ import annotations

import numpy as np


def kda_recurrent(q, k, v, g, beta, scale=None, state=None):
    """q, k [B, T, H, K]; v [B, T, HV, V]; g [B, T, HV, K]; beta [B, T, HV];
    state [B, HV, K, V] or None (zeros).  Returns (o [B, T, HV, V], S [B, HV, K, V]),
    float64."""
    f = lambda a: np.asarray(a, dtype=np.float64)  # noqa: E731
    q, k, v, g, beta = f(q), f(k), f(v), f(g), f(beta)
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    G = HV // H
    if scale is None:
        scale = K ** -0.5
    q = np.repeat(q, G, axis=2) * scale
    k = np.repeat(k, G, axis=2)
    S = np.zeros((B, HV, K, V)) if state is None else f(state).copy()
    o = np.zeros((B, T, HV, V))
    for i in range(T):
        S = S * np.exp(g[:, i])[..., None]
        ks = np.einsum("bhk,bhkv->bhv", k[:, i], S)
        S = S + np.einsum("bhk,bhv->bhkv", beta[:, i][..., None] * k[:, i], v[:, i] - ks)
        o[:, i] = np.einsum("bhk,bhkv->bhv", q[:, i], S)
    return o, S


def l2norm(x, eps: float = 1e-6):
    """Last-axis L2 normalisation (the q/k normalisation of attention_kda.py:101-102)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + eps)


def short_conv(x, w, k: int, state=None):
    """Causal depthwise convolution over time, then SiLU (ops.py:46-60): x [B, T, C],
    w [C, k] (the checkpoint's [C, 1, k]), state [B, k-1, C] (the previous k-1 inputs,
    oldest first) or None.  y[t, c] = sum_j w[c, j] xp[t + j, c] with xp = state ++ x.
    Returns (silu(y), the last k-1 rows of xp)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64).reshape(x.shape[-1], k)
    B, T, C = x.shape
    pad = np.zeros((B, k - 1, C)) if state is None else np.asarray(state, np.float64)
    xp = np.concatenate([pad, x], axis=1)
    y = np.zeros((B, T, C))
    for j in range(k):
        y += w[:, j] * xp[:, j:j + T, :]
    return y / (1.0 + np.exp(-y)), xp[:, -(k - 1):, :]


def gated_rmsnorm(x, w, g, eps):
    """FusedRMSNormGated with sigmoid (ops.py:36-39) over the last axis, float64."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * np.asarray(w, np.float64) / (1.0 + np.exp(-np.asarray(g, np.float64)))


def kda_layer(cfg, w: dict, x, state=None, conv=None):
    """KDAAttention.__call__ (attention_kda.py:94-115; k3ref/layers.py:116-136) in float64.
    ``w`` holds the checkpoint tensors named in attention_kda.py:30-33 (conv weights
    [C, 1, k]); x [B, T, hidden]; state [B, H, D, D]; conv (cq, ck, cv) each [B, k-1, C].
    Returns (out [B, T, hidden], state, (cq, ck, cv))."""
    f = {n: np.asarray(a, np.float64) for n, a in w.items()}
    x = np.asarray(x, np.float64)
    B, T, _ = x.shape
    H, D, K = cfg.kda_num_heads, cfg.kda_head_dim, cfg.kda_conv_size
    cv_in = (None, None, None) if conv is None else conv
    q, cq = short_conv(x @ f["q_proj.weight"].T, f["q_conv1d.weight"], K, cv_in[0])
    k, ck = short_conv(x @ f["k_proj.weight"].T, f["k_conv1d.weight"], K, cv_in[1])
    v, cv = short_conv(x @ f["v_proj.weight"].T, f["v_conv1d.weight"], K, cv_in[2])
    q, k = l2norm(q.reshape(B, T, H, D)), l2norm(k.reshape(B, T, H, D))
    v = v.reshape(B, T, H, D)
    g_raw = ((x @ f["f_a_proj.weight"].T) @ f["f_b_proj.weight"].T).reshape(B, T, H, D) + f["dt_bias"].reshape(H, D)
    a_exp = np.exp(f["A_log"][:H]).reshape(H, 1)
    g = cfg.kda_gate_lower_bound / (1.0 + np.exp(-(a_exp * g_raw)))
    beta = 1.0 / (1.0 + np.exp(-(x @ f["b_proj.weight"].T)))
    o, S = kda_recurrent(q, k, v, g, beta, D ** -0.5, state)
    og = (x @ f["g_proj.weight"].T).reshape(B, T, H, D)
    o = gated_rmsnorm(o, f["o_norm.weight"], og, cfg.rms_norm_eps)
    return o.reshape(B, T, H * D) @ f["o_proj.weight"].T, S, (cq, ck, cv)


def random_kda_weights(rng, cfg, scale: float = 0.02) -> dict:
    """Float32 checkpoint tensors at cfg's shapes (the recipe of
    tools/make_synthetic_k3.py:190-203: N(0, 0.02) projections, conv N(0, 0.3), A_log
    log U(1, 16) on the first H entries and zero after, dt_bias N(0, 1))."""
    H, D, K, hid = cfg.kda_num_heads, cfg.kda_head_dim, cfg.kda_conv_size, cfg.hidden_size
    P = H * D

    def W(*shape, s=scale):
        return (rng.standard_normal(shape) * s).astype(np.float32)

    a = np.zeros(D, np.float32)
    a[:H] = np.log(rng.uniform(1, 16, H))
    return {"q_proj.weight": W(P, hid), "k_proj.weight": W(P, hid), "v_proj.weight": W(P, hid),
            "g_proj.weight": W(P, hid), "o_proj.weight": W(hid, P),
            "q_conv1d.weight": W(P, 1, K, s=0.3), "k_conv1d.weight": W(P, 1, K, s=0.3),
            "v_conv1d.weight": W(P, 1, K, s=0.3), "f_a_proj.weight": W(D, hid), "f_b_proj.weight": W(P, D),
            "b_proj.weight": W(H, hid), "o_norm.weight": (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32),
            "A_log": a, "dt_bias": W(P, s=1.0)}
