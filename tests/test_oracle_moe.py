"""Pin the MoE oracle (CPU only).

Every check compares ``oracle/moe.py`` with something that does not share its code: torch's
softmax / sigmoid / topk as library routines, the router invariants of the reference's
``tests/test_k3ref_layers.py:113-127``, closed forms of the activations at chosen points,
and brute-force scalar loops over weights decoded by the independent C restatement
(``oracle/mxfp4_ref.c``).  Planted mistakes (weights gathered from the corrected scores,
gate and up swapped, a dropped renormalisation) must be caught.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import moe as omoe
from oracle import mxfp4 as om
from oracle import native

torch = pytest.importorskip("torch")


# ------------------------------------------------------------------------- routers
def test_softmax_route_matches_torch_library():
    rng = np.random.default_rng(21)
    x = rng.standard_normal((5, 96))
    wr = rng.standard_normal((40, 96)) * 0.3
    idx, w, probs, logits = omoe.route_softmax(x, wr, k=6)
    tl = torch.from_numpy(x) @ torch.from_numpy(wr).T
    tp = torch.softmax(tl, dim=-1)
    assert np.allclose(probs, tp.numpy(), rtol=1e-13, atol=0)
    tv, ti = torch.topk(tp, 6, dim=-1)
    assert np.array_equal(idx, ti.numpy())
    assert np.allclose(w, (tv / tv.sum(-1, keepdim=True)).numpy(), rtol=1e-13)
    assert np.allclose(w.sum(-1), 1.0, rtol=1e-14)
    # no renormalisation: weights are the probabilities themselves, times the scaling
    _, w2, _, _ = omoe.route_softmax(x, wr, k=6, renormalize=False, scaling=2.5)
    assert np.allclose(w2, 2.5 * tv.numpy(), rtol=1e-13)


def test_topk_ties_go_to_lower_index():
    s = np.array([[0.1, 0.5, 0.5, 0.2, 0.5, 0.0],
                  [1.0, 1.0, 1.0, 1.0, 1.0, 1.0]])
    assert omoe.topk_lowest_index(s, 2).tolist() == [[1, 2], [0, 1]]
    assert omoe.topk_lowest_index(s, 4).tolist() == [[1, 2, 4, 3], [0, 1, 2, 3]]


def _check_router_invariants(x, wr, bias, k, scaling, idx, w, raw, corrected):
    """The reference's router gates (tests/test_k3ref_layers.py:113-127)."""
    tl = torch.from_numpy(x) @ torch.from_numpy(wr).T
    traw = torch.sigmoid(tl).numpy()
    assert np.allclose(raw, traw, rtol=1e-13, atol=1e-300)
    assert np.allclose(corrected, traw + bias[None, :], rtol=1e-13)
    for t in range(x.shape[0]):
        assert len(set(idx[t].tolist())) == k                      # k distinct experts
        _, ti = torch.topk(torch.from_numpy(traw[t] + bias), k)     # selection on corrected
        assert sorted(idx[t].tolist()) == sorted(ti.tolist())
        g = traw[t][idx[t]]                                         # weights from RAW scores
        assert np.allclose(w[t], g / (g.sum() + 1e-20) * scaling, rtol=1e-13)
        assert math.isclose(w[t].sum(), scaling, rel_tol=1e-12)


def test_sigmoid_bias_route_invariants():
    rng = np.random.default_rng(22)
    x = rng.standard_normal((4, 64))
    wr = rng.standard_normal((48, 64)) * 0.2
    bias = rng.standard_normal(48) * 0.3      # large enough that it changes the selection
    idx, w, raw, corrected = omoe.route_sigmoid_bias(x, wr, bias, k=8, scaling=2.827)
    sel_raw = omoe.topk_lowest_index(raw, 8)
    assert any(sorted(a) != sorted(b) for a, b in zip(idx.tolist(), sel_raw.tolist()))
    _check_router_invariants(x, wr, bias, 8, 2.827, idx, w, raw, corrected)


def test_planted_router_mistake_is_caught():
    """Weights gathered from the corrected scores (a plausible slip) fail the gate."""
    rng = np.random.default_rng(23)
    x = rng.standard_normal((3, 32))
    wr = rng.standard_normal((24, 32)) * 0.2
    bias = rng.standard_normal(24) * 0.3
    idx, _, raw, corrected = omoe.route_sigmoid_bias(x, wr, bias, k=4)
    g = np.take_along_axis(corrected, idx, axis=-1)
    bad_w = g / (g.sum(-1, keepdims=True) + 1e-20)
    with pytest.raises(AssertionError):
        _check_router_invariants(x, wr, bias, 4, 1.0, idx, bad_w, raw, corrected)


# ------------------------------------------------------------------------- activations
def test_silu_closed_forms_and_torch():
    assert omoe.silu(np.array(0.0)) == 0.0
    assert math.isclose(float(omoe.silu(np.array(40.0))), 40.0, rel_tol=1e-15)
    assert abs(float(omoe.silu(np.array(-40.0)))) < 1e-15
    assert math.isclose(float(omoe.silu(np.array(1.0))), 1.0 / (1.0 + math.exp(-1.0)), rel_tol=1e-15)
    g = np.linspace(-12, 12, 97)
    # the oracle uses the overflow-free tanh form of the logistic; cancellation in 1 + tanh
    # for very negative g costs a few digits relative to torch's 1 / (1 + exp(-g))
    assert np.allclose(omoe.silu(g), torch.nn.functional.silu(torch.from_numpy(g)).numpy(), rtol=1e-9, atol=1e-300)
    u = np.linspace(-3, 3, 97)
    assert np.allclose(omoe.activation(g, u, "silu"), omoe.silu(g) * u, rtol=0, atol=0)


def test_situ_closed_forms():
    """beta*tanh(g/beta)*sigmoid(g) * lbeta*tanh(u/lbeta) (ops.py:17-28)."""
    beta, lbeta = 2.5, 3.0
    # g -> +inf: tanh -> 1, sigmoid -> 1, so the gate half saturates at beta
    assert math.isclose(float(omoe.situ(np.array(60.0), np.array(1.0), beta, None)), beta, rel_tol=1e-14)
    # g -> -inf: sigmoid -> 0
    assert abs(float(omoe.situ(np.array(-60.0), np.array(1.0), beta, None))) < 1e-20
    # u -> +inf with a linear beta saturates at lbeta; without one it stays linear
    assert math.isclose(float(omoe.situ(np.array(60.0), np.array(1e3), beta, lbeta)), beta * lbeta, rel_tol=1e-14)
    assert math.isclose(float(omoe.situ(np.array(60.0), np.array(7.0), beta, None)), beta * 7.0, rel_tol=1e-14)
    # small g: beta*tanh(g/beta) ~ g, so situ ~ silu(g) * u
    g = np.array(1e-4)
    assert math.isclose(float(omoe.situ(g, np.array(2.0), beta, None)), float(omoe.silu(g)) * 2.0, rel_tol=1e-8)
    gt, ut = torch.tensor(0.7, dtype=torch.float64), torch.tensor(-1.3, dtype=torch.float64)
    want = beta * torch.tanh(gt / beta) * torch.sigmoid(gt) * lbeta * torch.tanh(ut / lbeta)
    assert math.isclose(float(omoe.situ(np.array(0.7), np.array(-1.3), beta, lbeta)), float(want), rel_tol=1e-14)


# ------------------------------------------------------------------------- expert / layer
def _brute_expert(x, gate, up, down, kind="silu", beta=1.0, lbeta=None):
    """Scalar loops with math.fsum over weights decoded by the C restatement."""
    wg, wu, wd = (native.decode_f32(*p).astype(np.float64) for p in (gate, up, down))
    I, H = wg.shape
    act = []
    for i in range(I):
        g = math.fsum(float(x[h]) * wg[i, h] for h in range(H))
        u = math.fsum(float(x[h]) * wu[i, h] for h in range(H))
        if kind == "silu":
            act.append(g / (1.0 + math.exp(-g)) * u)
        else:
            a = beta * math.tanh(g / beta) / (1.0 + math.exp(-g))
            act.append(a * (lbeta * math.tanh(u / lbeta) if lbeta else u))
    return np.array([math.fsum(act[i] * wd[n, i] for i in range(I)) for n in range(H)])


@pytest.mark.parametrize("kind", ["silu", "situ"])
def test_expert_ffn_vs_brute_force(kind):
    native.build(force=False)
    rng = np.random.default_rng(24)
    H, I = 64, 32
    gate, up = om.random_mxfp4(rng, I, H, 122, 126), om.random_mxfp4(rng, I, H, 122, 126)
    down = om.random_mxfp4(rng, H, I, 122, 126)
    x = om.bf16_round(rng.standard_normal(H).astype(np.float32))
    got = omoe.expert_ffn(x[None, :], gate, up, down, kind=kind, beta=2.0, linear_beta=3.0 if kind == "situ" else None)[0][0]
    want = _brute_expert(x, gate, up, down, kind, 2.0, 3.0 if kind == "situ" else None)
    assert om.normwise_rel(got, want) < 1e-12
    # planted mistake: gate and up swapped
    swapped = omoe.expert_ffn(x[None, :], up, gate, down, kind=kind, beta=2.0)[0][0]
    assert om.normwise_rel(swapped, want) > 1e-2


def test_moe_layer_vs_token_slot_loop():
    """The oracle loops experts in ascending id; restate it token by token, slot by slot,
    with dense weights from the C decode, and with the shared expert added."""
    native.build(force=False)
    rng = np.random.default_rng(25)
    H, I, E, k, T = 64, 32, 6, 3, 4
    experts = [(om.random_mxfp4(rng, I, H, 122, 126), om.random_mxfp4(rng, I, H, 122, 126),
                om.random_mxfp4(rng, H, I, 122, 126)) for _ in range(E)]
    shared = tuple(rng.standard_normal(s) * 0.05 for s in ((I, H), (I, H), (H, I)))
    x = om.bf16_round(rng.standard_normal((T, H)).astype(np.float32)).astype(np.float64)
    wr = rng.standard_normal((E, H)) * 0.1
    idx, w, _, _ = omoe.route_softmax(x, wr, k)
    got = omoe.moe_layer(x, idx, w, experts, shared=shared)
    want = np.zeros((T, H))
    for t in range(T):
        for j in range(k):
            gate, up, down = experts[idx[t, j]]
            wg, wu, wd = (native.decode_f32(*p).astype(np.float64) for p in (gate, up, down))
            g, u = wg @ x[t], wu @ x[t]
            want[t] += w[t, j] * (wd @ (g / (1 + np.exp(-g)) * u))
        g, u = shared[0] @ x[t], shared[1] @ x[t]
        want[t] += shared[2] @ (g / (1 + np.exp(-g)) * u)
    assert om.normwise_rel(got, want) < 1e-12
    # planted mistake: the renormalisation dropped
    w_raw = np.take_along_axis(omoe.route_softmax(x, wr, k, renormalize=False)[2], idx, axis=-1)
    bad = omoe.moe_layer(x, idx, w_raw, experts, shared=shared)
    assert om.normwise_rel(bad, want) > 1e-2


# ------------------------------------------------------------------------- latent layer
def _latent_case(seed=31, H=96, L=64, I=32, E=8, k=3, T=3, Is=40):
    rng = np.random.default_rng(seed)
    experts = [(om.random_mxfp4(rng, I, L, 122, 126), om.random_mxfp4(rng, I, L, 122, 126),
                om.random_mxfp4(rng, L, I, 122, 126)) for _ in range(E)]
    shared = tuple(rng.standard_normal(s) * 0.05 for s in ((Is, H), (Is, H), (H, Is)))
    x = rng.standard_normal((T, H))
    wr = rng.standard_normal((E, H)) * 0.1
    bias = rng.standard_normal(E) * 0.05
    down = rng.standard_normal((L, H)) * 0.1
    up = rng.standard_normal((H, L)) * 0.1
    norm_w = 1.0 + 0.1 * rng.standard_normal(L)
    return x, wr, bias, down, up, norm_w, experts, shared, k


def test_rmsnorm_closed_form_and_torch():
    """rms_norm of torch (a library routine) and a constant vector (x / |x_i| * w)."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 33))
    w = rng.standard_normal(33)
    want = torch.nn.functional.rms_norm(torch.from_numpy(x), (33,), torch.from_numpy(w), eps=1e-5).numpy()
    assert np.allclose(omoe.rmsnorm(x, w, 1e-5), want, rtol=1e-12, atol=1e-12)
    c = np.full((1, 8), -3.0)
    assert np.allclose(omoe.rmsnorm(c, np.arange(8.0), 0.0), -np.arange(8.0)[None, :], rtol=1e-14)


def test_latent_layer_reduces_to_normalised_plain_layer():
    """Identity down/up projections and unit norm weights: the latent layer is
    rmsnorm(plain routed layer) + shared, routed by the same sigmoid + bias router."""
    x, wr, bias, _, _, _, experts, shared, k = _latent_case(H=64, L=64)
    eye = np.eye(64)
    got, idx, w = omoe.latent_moe(x, wr, bias, eye, eye, np.ones(64), experts, shared, k, eps=1e-6)
    r_idx, r_w, _, _ = omoe.route_sigmoid_bias(x, wr, bias, k)
    assert np.array_equal(idx, r_idx) and np.allclose(w, r_w, rtol=1e-14)
    plain = omoe.moe_layer(x, idx, w, experts, None, "situ")
    want = plain / np.sqrt((plain * plain).mean(axis=-1, keepdims=True) + 1e-6)
    want = want + omoe.dense_ffn(x, *shared, kind="situ")[0]
    assert om.normwise_rel(got, want) < 1e-12


def test_latent_layer_invariants_and_planted_mistake():
    """The routed scaling factor cancels in the normalisation (eps = 0); the layer is
    linear in the up projection; normalising after the up projection (a plausible slip)
    changes the result."""
    x, wr, bias, down, up, norm_w, experts, shared, k = _latent_case()
    a = omoe.latent_moe(x, wr, bias, down, up, norm_w, experts, shared, k, scaling=1.0, eps=0.0)[0]
    b = omoe.latent_moe(x, wr, bias, down, up, norm_w, experts, shared, k, scaling=2.5, eps=0.0)[0]
    assert om.normwise_rel(a, b) < 1e-12
    sh = omoe.dense_ffn(x, *shared, kind="situ")[0]
    c = omoe.latent_moe(x, wr, bias, down, 3.0 * up, norm_w, experts, shared, k, eps=0.0)[0]
    assert om.normwise_rel(c - sh, 3.0 * (a - sh)) < 1e-12
    idx, w, _, _ = omoe.route_sigmoid_bias(x, wr, bias, k)
    y = omoe.moe_layer(x @ down.T, idx, w, experts, None, "situ") @ up.T
    bad = omoe.rmsnorm(y, np.ones(up.shape[0]), 0.0) + sh
    assert om.normwise_rel(bad, a) > 1e-2
