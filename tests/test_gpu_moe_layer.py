"""GPU parity of the routed MoE layer (router + top-k + routed experts + shared expert)
against the fp64 oracle, through the LatentMoE-shaped dispatcher."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_layer(seed, H, I, E, k, Is=0, distinct=None, router="softmax", act="silu", beta=1.0, lbeta=None,
               renorm=True, scaling=1.0):
    """Random layer.  `distinct` experts are generated and expert e aliases e % distinct,
    which exercises the device pointer table at large E with little memory."""
    from k3hip.moe import MoEConfig
    rng = np.random.default_rng(seed)
    D = distinct or E
    experts_np = [(om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, H, I))
                  for _ in range(D)]
    experts_dev = [tuple(tuple(torch.from_numpy(a).to(DEV) for a in pair) for pair in ex) for ex in experts_np]
    router_w = om.bf16_round((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    w = {"gate.weight": torch.from_numpy(router_w).to(DEV).to(torch.bfloat16)}
    bias = None
    if router == "sigmoid_bias":
        bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
        w["gate.e_score_correction_bias"] = torch.from_numpy(bias).to(DEV)
    shared_np = None
    if Is:
        shared_np = tuple(om.bf16_round((rng.standard_normal(s) * 0.02).astype(np.float32))
                          for s in ((Is, H), (Is, H), (H, Is)))
        for name, a in zip(("gate", "up", "down"), shared_np):
            w[f"shared_experts.{name}_proj.weight"] = torch.from_numpy(a).to(DEV).to(torch.bfloat16)
    which_ix = {"w1": 0, "w3": 1, "w2": 2}

    def source(layer, e, which):
        return experts_dev[e % D][which_ix[which]]

    cfg = MoEConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, num_experts_per_token=k,
                    shared_intermediate_size=Is, moe_renormalize=renorm, routed_scaling_factor=scaling,
                    router=router, activation=act, situ_beta=beta, situ_linear_beta=lbeta)
    oracle_experts = {e: experts_np[e % D] for e in range(E)}
    return cfg, w, source, router_w, bias, oracle_experts, shared_np


def oracle_layer(x32, router_w, bias, experts, shared, cfg):
    if cfg.router == "softmax":
        idx, wts, raw, _ = omoe.route_softmax(x32, router_w, cfg.num_experts_per_token, cfg.moe_renormalize,
                                              cfg.routed_scaling_factor)
        corrected = raw
    else:
        idx, wts, raw, corrected = omoe.route_sigmoid_bias(x32, router_w, bias, cfg.num_experts_per_token,
                                                           cfg.moe_renormalize, cfg.routed_scaling_factor)
    y = omoe.moe_layer(x32, idx, wts, experts, shared, kind=cfg.activation, beta=cfg.situ_beta,
                       linear_beta=cfg.situ_linear_beta)
    return y, idx, wts, raw, corrected


def topk_margin(sel, k):
    s = np.sort(np.asarray(sel, np.float64).ravel())[::-1]
    return s[k - 1] - s[k]


CASES = [
    # H, I, E, k, Is, distinct, router, act, xdt
    (1024, 256, 16, 4, 256, None, "softmax", "silu", torch.bfloat16),
    (1024, 256, 16, 4, 0, None, "softmax", "silu", torch.float32),
    (2048, 384, 64, 8, 512, 8, "sigmoid_bias", "situ", torch.bfloat16),
    (7168, 2048, 384, 8, 2048, 12, "softmax", "silu", torch.bfloat16),
    (3584, 3072, 96, 8, 0, 6, "sigmoid_bias", "situ", torch.bfloat16),
    (2048, 4096, 32, 16, 0, 8, "sigmoid_bias", "situ", torch.bfloat16),
    # a shared expert wide enough that L1's grid takes more than one round of blocks (the
    # launch without the up-row delay)
    (2048, 512, 64, 4, 6144, 8, "softmax", "silu", torch.bfloat16),
]


@pytest.mark.parametrize("H,I,E,k,Is,distinct,router,act,xdt", CASES)
def test_layer_matches_oracle(H, I, E, k, Is, distinct, router, act, xdt):
    from k3hip.moe import RoutedMoE
    beta, lbeta = (4.0, 25.0) if act == "situ" else (1.0, None)
    cfg, w, source, router_w, bias, experts, shared = make_layer(H + E, H, I, E, k, Is, distinct, router, act,
                                                                 beta, lbeta)
    moe = RoutedMoE(cfg, 1, w, source)
    rng = np.random.default_rng(E)
    x32 = rng.standard_normal((1, H)).astype(np.float32)
    if xdt == torch.bfloat16:
        x32 = om.bf16_round(x32)
    x = torch.from_numpy(x32).to(DEV).to(xdt)
    y_want, idx, wts, raw, corrected = oracle_layer(x32, router_w, bias, experts, shared, cfg)
    sel = corrected if router == "sigmoid_bias" else raw
    assert topk_margin(sel, k) > 1e-5, "seed gives a near-tie at the top-k boundary"
    y, r = moe(x, return_router=True)
    got_idx = r.expert_indices.cpu().numpy()
    assert np.array_equal(np.sort(got_idx, -1), np.sort(idx, -1))
    order = np.argsort(got_idx[0])
    assert np.allclose(r.expert_weights.cpu().numpy()[0][order], wts[0][np.argsort(idx[0])], rtol=0, atol=1e-5)
    assert np.allclose(r.raw_scores.cpu().numpy(), raw, rtol=1e-4, atol=1e-6)
    assert om.normwise_rel(y.cpu().numpy(), y_want) < 2e-5


def test_layer_full_shape_every_expert_distinct():
    """The 384-expert top-8 layer at full size with every expert distinct (9 GB of weights
    drawn on the device; only the selected experts are copied to the host for the oracle),
    a bf16 shared expert, three tokens in a row through one module, then four and eight
    tokens at once through the multi-token decode."""
    from k3hip.moe import MoEConfig, RoutedMoE
    H, I, E, k, Is = 7168, 2048, 384, 8, 2048
    g = torch.Generator(device=DEV)
    g.manual_seed(384)

    def mx(n, kk):
        return (torch.randint(0, 256, (n, kk // 2), dtype=torch.uint8, device=DEV, generator=g),
                torch.randint(118, 131, (n, kk // 32), dtype=torch.uint8, device=DEV, generator=g))

    experts = [(mx(I, H), mx(I, H), mx(H, I)) for _ in range(E)]
    rng = np.random.default_rng(385)
    router_w = om.bf16_round((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    shared = tuple(om.bf16_round((rng.standard_normal(sh) * 0.02).astype(np.float32))
                   for sh in ((Is, H), (Is, H), (H, Is)))
    w = {"gate.weight": torch.from_numpy(router_w).to(DEV).to(torch.bfloat16)}
    for name, a in zip(("gate", "up", "down"), shared):
        w[f"shared_experts.{name}_proj.weight"] = torch.from_numpy(a).to(DEV).to(torch.bfloat16)
    cfg = MoEConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, num_experts_per_token=k,
                    shared_intermediate_size=Is, router="softmax", activation="silu")
    which = {"w1": 0, "w3": 1, "w2": 2}
    moe = RoutedMoE(cfg, 1, w, lambda layer, e, wh: experts[e][which[wh]])
    seen = set()
    for t in range(3):
        x32 = om.bf16_round(rng.standard_normal((1, H)).astype(np.float32))
        idx, wts, raw, _ = omoe.route_softmax(x32, router_w, k, True, 1.0)
        assert topk_margin(raw, k) > 1e-5, "seed gives a near-tie at the top-k boundary"
        sel = {int(e): tuple(tuple(a.cpu().numpy() for a in pair) for pair in experts[int(e)]) for e in idx[0]}
        y_want = omoe.moe_layer(x32, idx, wts, sel, shared)
        y, r = moe(torch.from_numpy(x32).to(DEV).to(torch.bfloat16), return_router=True)
        assert np.array_equal(np.sort(r.expert_indices.cpu().numpy(), -1), np.sort(idx, -1))
        rel = om.normwise_rel(y.cpu().numpy(), y_want)
        print(f"token {t}: experts {sorted(sel)} rel={rel:.3e}")
        assert rel < 2e-5
        seen.update(sel)
    assert len(seen) > 16  # distinct weights behind distinct experts, not a few aliased sets
    # four and eight tokens at once: the multi-token decode (k3_moe_layer_decode_multi), each
    # selected expert read once for all its tokens, the shared expert on the side stream
    workers = max(1, min(16, len(os.sched_getaffinity(0))))
    for T in (4, 8):
        x32 = om.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
        idx, wts, raw, _ = omoe.route_softmax(x32, router_w, k, True, 1.0)
        assert min(topk_margin(raw[t], k) for t in range(T)) > 1e-5, "seed gives a near-tie at the top-k boundary"
        sel = {int(e): tuple(tuple(a.cpu().numpy() for a in pair) for pair in experts[int(e)]) for e in np.unique(idx)}
        y_want = omoe.moe_layer(x32, idx, wts, sel, shared, workers=workers)
        y, r = moe(torch.from_numpy(x32).to(DEV).to(torch.bfloat16), return_router=True)
        assert np.array_equal(np.sort(r.expert_indices.cpu().numpy(), -1), np.sort(idx, -1))
        rel = om.normwise_rel(y.cpu().numpy(), y_want)
        print(f"{T} tokens: {len(sel)} distinct experts rel={rel:.3e}")
        assert rel < 2e-5


def test_route_only_matches_layer_record_and_invariants():
    """The invariants of tests/test_k3ref_layers.py:113-127 on the sigmoid+bias router:
    k distinct experts, weights renormalise to the scaling factor, selection follows the
    corrected scores, weights come from the raw scores."""
    from k3hip.moe import RoutedMoE
    cfg, w, source, *_ = make_layer(3, 1024, 256, 64, 8, 0, 4, "sigmoid_bias", "silu", scaling=2.5)
    moe = RoutedMoE(cfg, 0, w, source)
    x = torch.randn(3, 1024, device=DEV).to(torch.bfloat16)
    r = moe.route(x)
    idx = r.expert_indices
    assert all(len(set(row.tolist())) == 8 for row in idx)
    assert torch.allclose(r.expert_weights.sum(-1), torch.full((3,), 2.5, device=idx.device), atol=1e-5)
    assert torch.equal(idx.sort(-1).values, r.corrected_scores.topk(8, -1).indices.sort(-1).values)
    raw_k = r.raw_scores.gather(1, idx)
    assert torch.allclose(raw_k / raw_k.sum(-1, keepdim=True) * 2.5, r.expert_weights, atol=1e-6)
    # the layer kernel's own records (its in-kernel router rows) against route(), whose logits
    # come from one GEMM over all tokens: same experts, weights to fp32 accumulation-order noise
    _, r2 = moe(x, return_router=True)
    assert torch.equal(r2.expert_indices, idx)
    assert torch.allclose(r2.expert_weights, r.expert_weights, rtol=1e-5, atol=1e-7)


def test_layer_deterministic_and_graph_replay():
    from k3hip.moe import RoutedMoE
    cfg, w, source, *_ = make_layer(11, 2048, 512, 32, 8, 512, 8)
    moe = RoutedMoE(cfg, 0, w, source)
    xs = [torch.randn(1, 2048, device=DEV).to(torch.bfloat16) for _ in range(3)]
    ref = [moe(x).clone() for x in xs]
    for _ in range(5):
        for x, r in zip(xs, ref):
            assert torch.equal(moe(x), r)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [moe(x) for x in xs]
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o, r)
        assert torch.equal(moe(xs[0]), ref[0])   # eager work between replays


def test_layer_multi_token_and_unfused_expert():
    from k3hip.moe import RoutedMoE
    cfg, w, source, router_w, bias, experts, shared = make_layer(5, 1024, 256, 16, 4, 256)
    moe = RoutedMoE(cfg, 0, w, source)
    x32 = om.bf16_round(np.random.default_rng(1).standard_normal((3, 1024)).astype(np.float32))
    y = moe(torch.from_numpy(x32).to(DEV).to(torch.bfloat16)).cpu().numpy()
    for t in range(3):
        want = oracle_layer(x32[t:t + 1], router_w, bias, experts, shared, cfg)[0]
        assert om.normwise_rel(y[t:t + 1], want) < 2e-5
    # the fused=False debug path: bf16-decoded weights, fp32 matmuls
    h = torch.from_numpy(x32[:1]).to(DEV)
    ref_moe = RoutedMoE(cfg, 0, w, source, fused=False)
    a = ref_moe.expert_forward(h, 3).cpu().numpy()
    b = moe.expert_forward(h, 3).cpu().numpy()
    want = omoe.expert_ffn(x32[:1], *experts[3])[0]
    assert om.normwise_rel(a, want) < 1e-4 and om.normwise_rel(b, want) < 1e-5


def test_layer_counter_bytes_garbage():
    """Arrival counters holding garbage: L2 zeroes L3's range counters inside the call, so a
    layer whose workspace starts with garbage there is exact on its first call; garbage in
    L1's router counter is cleared by the first call (L2 zeroes it too), so the second call
    is exact."""
    from k3hip.moe import RoutedMoE
    cfg, w, source, router_w, bias, experts, shared = make_layer(21, 2048, 512, 64, 8, 512, 8)
    moe = RoutedMoE(cfg, 0, w, source)
    x32 = om.bf16_round(np.random.default_rng(22).standard_normal((1, 2048)).astype(np.float32))
    x = torch.from_numpy(x32).to(DEV).to(torch.bfloat16)
    want = oracle_layer(x32, router_w, bias, experts, shared, cfg)[0]
    moe(x)                                            # workspace exists
    ws = moe._workspace()
    ctr = ws[:4096].view(torch.int32)
    ctr[1:].fill_(0x5A5A5A5A)                         # every L3 range counter word
    assert om.normwise_rel(moe(x).cpu().numpy(), want) < 2e-5
    ranges = -(-2048 // 56)                           # L3 row ranges at I = 512 (56 rows each)
    assert int(ctr[1:1 + ranges].abs().max()) == 0
    ctr[0] = 7                                        # L1's router counter
    moe(x)
    assert int(ctr[0]) == 0
    assert om.normwise_rel(moe(x).cpu().numpy(), want) < 2e-5


@pytest.mark.parametrize("router", ["softmax", "sigmoid_bias"])
def test_route_only_with_garbage_counter(router):
    """k3_moe_route (router + top-k only) on a workspace whose router arrival counter holds
    garbage: the call resets the counter itself, so its first call already writes the
    oracle's selection and weights, and it leaves the counter at zero."""
    import ctypes

    from k3hip import _lib
    from k3hip import _torch as T
    H, E, k = 2048, 64, 6
    rng = np.random.default_rng(31 + len(router))
    router_w = om.bf16_round((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    kind = _lib.K3_ROUTE_SOFTMAX if router == "softmax" else _lib.K3_ROUTE_SIGMOID_BIAS
    rw = torch.from_numpy(router_w).to(DEV).to(torch.bfloat16)
    bd = torch.from_numpy(bias).to(DEV) if router == "sigmoid_bias" else None
    nbytes = int(_lib.lib().k3_moe_layer_workspace_size(H, 128, 0, E, k))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    off = (ctypes.c_int64 * 8)()
    _lib.call("k3_moe_layer_workspace_offsets", H, 128, 0, E, k, off)
    for garbage in (0x5A5A5A5A, 3, 0):
        x32 = om.bf16_round(rng.standard_normal((1, H)).astype(np.float32))
        x = torch.from_numpy(x32).to(DEV).to(torch.bfloat16)
        ws[:4].view(torch.int32).fill_(garbage)
        _lib.call("k3_moe_route", T.ptr(x), _lib.K3_BF16, T.ptr(rw), T.ptr(bd), kind, 1, 2.5, H, E, k,
                  T.ptr(ws), ws.numel(), T.stream(x))
        torch.cuda.synchronize()
        if router == "softmax":
            idx, wts, raw, _ = omoe.route_softmax(x32, router_w, k, True, 2.5)
        else:
            idx, wts, raw, corr = omoe.route_sigmoid_bias(x32, router_w, bias, k, True, 2.5)
        got_idx = ws[off[3]:off[3] + 4 * k].view(torch.int32).cpu().numpy()
        got_w = ws[off[4]:off[4] + 4 * k].view(torch.float32).cpu().numpy()
        got_raw = ws[off[1]:off[1] + 4 * E].view(torch.float32).cpu().numpy()
        assert np.array_equal(got_idx, idx[0]), (garbage, got_idx, idx[0])
        assert np.allclose(got_w, wts[0], rtol=1e-5, atol=1e-7)
        assert np.allclose(got_raw, raw[0], rtol=1e-4, atol=1e-7)
        assert int(ws[:4].view(torch.int32).item()) == 0
