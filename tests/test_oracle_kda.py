"""Pin the KDA recurrence oracle (CPU only): scalar loops, the delta rule's defining
property, closed forms at a zero state and at beta = 0, step-by-step == multi-step, and
planted mistakes."""
from __future__ import annotations

import numpy as np

from oracle import kda as okda


def _inputs(rng, B=1, T=3, H=2, HV=2, K=8, V=6):
    q = okda.l2norm(rng.standard_normal((B, T, H, K)))
    k = okda.l2norm(rng.standard_normal((B, T, H, K)))
    v = rng.standard_normal((B, T, HV, V))
    g = -5.0 / (1.0 + np.exp(-rng.standard_normal((B, T, HV, K))))     # the gate's range (-5, 0)
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, HV))))
    S0 = rng.standard_normal((B, HV, K, V))
    return q, k, v, g, beta, S0


def _loops(q, k, v, g, beta, scale, S0):
    B, T, H, K = q.shape
    HV, V = v.shape[2], v.shape[3]
    G = HV // H
    S = S0.copy()
    o = np.zeros((B, T, HV, V))
    for b in range(B):
        for i in range(T):
            for h in range(HV):
                hq = h // G
                for a in range(K):
                    for c in range(V):
                        S[b, h, a, c] *= np.exp(g[b, i, h, a])
                ks = [sum(k[b, i, hq, a] * S[b, h, a, c] for a in range(K)) for c in range(V)]
                for a in range(K):
                    for c in range(V):
                        S[b, h, a, c] += beta[b, i, h] * k[b, i, hq, a] * (v[b, i, h, c] - ks[c])
                for c in range(V):
                    o[b, i, h, c] = sum(scale * q[b, i, hq, a] * S[b, h, a, c] for a in range(K))
    return o, S


def test_matches_scalar_loops_including_grouped_heads():
    rng = np.random.default_rng(0)
    for H, HV in ((2, 2), (1, 3)):
        q, k, v, g, beta, S0 = _inputs(rng, B=2, T=3, H=H, HV=HV)
        o, S = okda.kda_recurrent(q, k, v, g, beta, 0.37, S0)
        lo, lS = _loops(q, k, v, g, beta, 0.37, S0)
        assert np.allclose(o, lo, rtol=1e-13, atol=1e-13) and np.allclose(S, lS, rtol=1e-13, atol=1e-13)


def test_delta_rule_writes_v_at_a_unit_key():
    """beta = 1, |k| = 1: k . S_new = k . S' + (k . k)(v - k . S') = v, for any state and
    decay.  Taking the delta on the undecayed state breaks it."""
    rng = np.random.default_rng(1)
    q, k, v, g, beta, S0 = _inputs(rng, T=1, K=16, V=16)
    k = k / np.linalg.norm(k, axis=-1, keepdims=True)
    beta = np.ones_like(beta)
    _, S = okda.kda_recurrent(q, k, v, g, beta, None, S0)
    assert np.allclose(np.einsum("bhk,bhkv->bhv", k[:, 0], S), v[:, 0], rtol=0, atol=1e-12)
    # planted: delta on the state before the decay
    Sd = S0 * np.exp(g[:, 0])[..., None]
    bad = Sd + np.einsum("bhk,bhv->bhkv", k[:, 0], v[:, 0] - np.einsum("bhk,bhkv->bhv", k[:, 0], S0))
    assert not np.allclose(np.einsum("bhk,bhkv->bhv", k[:, 0], bad), v[:, 0], atol=1e-6)


def test_zero_state_and_pure_decay_closed_forms():
    rng = np.random.default_rng(2)
    q, k, v, g, beta, S0 = _inputs(rng, T=1, K=8, V=5)
    o, S = okda.kda_recurrent(q, k, v, g, beta, 0.5, None)
    want_S = beta[:, 0][..., None, None] * np.einsum("bhk,bhv->bhkv", k[:, 0], v[:, 0])
    assert np.allclose(S, want_S, rtol=1e-14, atol=0)
    qk = (q[:, 0] * k[:, 0]).sum(-1)
    assert np.allclose(o[:, 0], 0.5 * (beta[:, 0] * qk)[..., None] * v[:, 0], rtol=1e-13)
    # a read-out taken before the update would return 0 here
    assert np.abs(o).max() > 1e-3
    o, S = okda.kda_recurrent(q, k, v, g, np.zeros_like(beta), 0.5, S0)
    Sd = S0 * np.exp(g[:, 0])[..., None]
    assert np.allclose(S, Sd, rtol=1e-15) and np.allclose(o[:, 0], 0.5 * np.einsum("bhk,bhkv->bhv", q[:, 0], Sd))


def test_steps_compose():
    rng = np.random.default_rng(3)
    q, k, v, g, beta, S0 = _inputs(rng, T=6, K=8, V=8)
    o, S = okda.kda_recurrent(q, k, v, g, beta, None, S0)
    St = S0
    for i in range(6):
        oi, St = okda.kda_recurrent(q[:, i:i + 1], k[:, i:i + 1], v[:, i:i + 1], g[:, i:i + 1], beta[:, i:i + 1],
                                    None, St)
        assert np.allclose(oi[:, 0], o[:, i], rtol=1e-13, atol=1e-14)
    assert np.allclose(St, S, rtol=1e-13, atol=1e-14)
