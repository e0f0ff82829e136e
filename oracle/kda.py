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
