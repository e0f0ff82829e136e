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


class _Cfg:
    hidden_size, kda_num_heads, kda_head_dim, kda_conv_size = 48, 2, 8, 4
    kda_gate_lower_bound, rms_norm_eps = -5.0, 1e-5


def test_short_conv_matches_numpy_correlate():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 7, 5))
    w = rng.standard_normal((5, 1, 4))
    st = rng.standard_normal((1, 3, 5))
    y, new = okda.short_conv(x, w, 4, st)
    xp = np.concatenate([st, x], axis=1)
    for c in range(5):
        pre = np.correlate(xp[0, :, c], w[c, 0], mode="valid")        # library routine
        assert np.allclose(y[0, :, c], pre / (1 + np.exp(-pre)), rtol=1e-14)
    assert np.array_equal(new[0], xp[0, -3:])


def test_gated_rmsnorm_and_l2norm_closed_forms():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 16))
    w = rng.standard_normal(16)
    y = okda.gated_rmsnorm(x, w, np.zeros_like(x), 0.0)           # sigmoid(0) = 1/2
    assert np.allclose(y, 0.5 * w * x / np.sqrt((x * x).mean(-1, keepdims=True)), rtol=1e-14)
    n = okda.l2norm(x, eps=0.0)
    assert np.allclose((n * n).sum(-1), 1.0, rtol=1e-14)


def test_layer_prefill_equals_incremental_and_gate_range():
    """The reference's KDA state gate (tests/test_k3ref_layers.py:150-168): one call over
    T tokens equals T single-token calls carrying the recurrent and convolution states."""
    cfg = _Cfg()
    rng = np.random.default_rng(6)
    w = okda.random_kda_weights(rng, cfg, scale=0.2)
    x = rng.standard_normal((1, 6, cfg.hidden_size))
    full, S_full, conv_full = okda.kda_layer(cfg, w, x)
    st, cv, outs = None, None, []
    for t in range(6):
        o, st, cv = okda.kda_layer(cfg, w, x[:, t:t + 1], st, cv)
        outs.append(o)
    assert np.allclose(np.concatenate(outs, axis=1), full, rtol=1e-12, atol=1e-13)
    assert np.allclose(st, S_full, rtol=1e-12, atol=1e-13)
    assert all(np.allclose(a, b) for a, b in zip(cv, conv_full))
    # the decay gate stays in (lower_bound, 0)
    f = {n: np.asarray(a, np.float64) for n, a in w.items()}
    g_raw = (x @ f["f_a_proj.weight"].T) @ f["f_b_proj.weight"].T
    g = -5.0 / (1 + np.exp(-(np.repeat(np.exp(f["A_log"][:2]), 8) * (g_raw + f["dt_bias"]))))
    assert np.all((g > -5.0) & (g < 0.0))
