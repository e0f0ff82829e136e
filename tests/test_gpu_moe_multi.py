"""GPU parity of the multi-token decode path (k3_moe_routed_decode: 2..8 tokens, every
expert any token selects read once) against the fp64 oracle.

Tolerance: normwise max-relative error 2e-5 (fp32 accumulation of exact MXFP4 x bf16
products, as the batch-1 layer); the K3 latent wrapper's bar is the decode path's, 1e-5,
except where the BLAS latent state can round one ulp away from the oracle's.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2e-5


def host_experts(rng, E, H, I):
    ex_np = [(om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, H, I)) for _ in range(E)]
    ex_dev = [tuple(tuple(torch.from_numpy(a).to(DEV) for a in pair) for pair in ex) for ex in ex_np]
    return ex_np, ex_dev


def device_experts(E, H, I, seed):
    """E distinct experts drawn on the device (scale bytes 118..130)."""
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)

    def mx(n, kk):
        return (torch.randint(0, 256, (n, kk // 2), dtype=torch.uint8, device=DEV, generator=g),
                torch.randint(118, 131, (n, kk // 32), dtype=torch.uint8, device=DEV, generator=g))

    return [(mx(I, H), mx(I, H), mx(H, I)) for _ in range(E)]


class HostExperts:
    """experts[e] for the oracle, copied from the device on access."""

    def __init__(self, ex_dev):
        self.ex_dev = ex_dev

    def __getitem__(self, e):
        return tuple(tuple(a.cpu().numpy() for a in pair) for pair in self.ex_dev[e])


def table_of(ex_dev):
    return torch.tensor([[t.data_ptr() for pair in ex for t in pair] for ex in ex_dev], dtype=torch.int64,
                        device=DEV)


def distinct_routing(rng, T, E, k):
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    return idx, w / w.sum(axis=1, keepdims=True)


def run(x, idx, w, ex_dev, I, act="silu", beta=1.0, lbeta=None, out_dtype=torch.float32, validate=True):
    from k3hip.moe import moe_routed_decode
    y = moe_routed_decode(x, torch.from_numpy(idx).to(DEV), torch.from_numpy(w).to(DEV), table_of(ex_dev), I, act,
                          beta, lbeta, out_dtype=out_dtype, validate=validate)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


CASES = [
    # T, H, I, E, k, routing, act, x dtype
    (2, 512, 256, 16, 4, "distinct", "silu", torch.bfloat16),
    (4, 1024, 384, 32, 8, "distinct", "situ", torch.bfloat16),
    (8, 2048, 512, 64, 8, "hot", "silu", torch.bfloat16),     # expert 5 in every token
    (8, 768, 256, 8, 8, "all", "silu", torch.bfloat16),       # every token takes every expert
    (3, 1024, 3072, 24, 16, "distinct", "situ", torch.bfloat16),  # I = 3072: half-group pieces
    (5, 2048, 4096, 16, 4, "distinct", "silu", torch.bfloat16),   # I = 4096: two pieces per lane
    (4, 8192, 256, 16, 4, "distinct", "silu", torch.bfloat16),    # H = 8192: four groups per lane
    (4, 1024, 256, 16, 4, "hot", "silu", torch.float32),          # fp32 x, two tokens per LDS batch
    (7, 7168, 256, 16, 6, "hot", "situ", torch.float32),
    (1, 1024, 256, 16, 4, "distinct", "silu", torch.bfloat16),
]


@pytest.mark.parametrize("T,H,I,E,k,routing,act,xdt", CASES)
def test_routed_decode_matches_oracle(T, H, I, E, k, routing, act, xdt):
    rng = np.random.default_rng(7000 + T * 31 + H + I)
    ex_np, ex_dev = host_experts(rng, E, H, I)
    if routing == "all":
        idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
        w = rng.random((T, k)).astype(np.float32)
    else:
        idx, w = distinct_routing(rng, T, E, k)
        if routing == "hot":
            for t in range(T):
                if 5 not in idx[t]:
                    idx[t, 0] = 5
    x32 = rng.standard_normal((T, H)).astype(np.float32)
    if xdt == torch.bfloat16:
        x32 = om.bf16_round(x32)
    beta, lbeta = (1.5, 3.0) if act == "situ" else (1.0, None)
    got = run(torch.from_numpy(x32).to(DEV).to(xdt), idx, w, ex_dev, I, act, beta, lbeta)
    want = omoe.moe_layer(x32, idx, w, {e: ex_np[e] for e in range(E)}, None, kind=act, beta=beta,
                          linear_beta=lbeta)
    rel = om.normwise_rel(got, want)
    print(f"T={T} H={H} I={I} E={E} k={k} {routing} {xdt}: {len(np.unique(idx))} experts, rel={rel:.3e}")
    assert rel <= TOL, rel


def test_routed_decode_full_shape_every_expert_distinct():
    """The 384-expert top-8 benchmark shape (hidden 7168, intermediate 2048) with all 384
    experts distinct on the device, four tokens; bit-identical on a second call; bf16 output
    is the fp32 output rounded."""
    T, H, I, E, k = 4, 7168, 2048, 384, 8
    ex_dev = device_experts(E, H, I, seed=4004)
    rng = np.random.default_rng(4004)
    idx, w = distinct_routing(rng, T, E, k)
    shared_e = next(int(e) for e in idx[0] if e not in idx[1])
    idx[1, 3] = shared_e                       # one expert shared by two tokens
    x = torch.from_numpy(om.bf16_round(rng.standard_normal((T, H)).astype(np.float32))).to(DEV).to(torch.bfloat16)
    got = run(x, idx, w, ex_dev, I)
    assert np.array_equal(got, run(x, idx, w, ex_dev, I))
    assert np.array_equal(run(x, idx, w, ex_dev, I, out_dtype=torch.bfloat16), om.bf16_round(got))
    workers = max(1, min(16, len(os.sched_getaffinity(0))))
    want = omoe.moe_layer(x.float().cpu().numpy(), idx, w, HostExperts(ex_dev), workers=workers)
    rel = om.normwise_rel(got, want)
    print(f"full shape T={T}: {len(np.unique(idx))} experts, rel={rel:.3e}")
    assert rel <= TOL, rel


def test_routed_decode_duplicate_and_invalid_ids():
    """A token listing one expert twice is gathered once with its first slot's weight (the
    reference's list.index, moe.py:121-122); unvalidated ids outside 0..E-1 contribute
    nothing; validated ones raise."""
    T, H, I, E, k = 3, 512, 256, 8, 4
    rng = np.random.default_rng(77)
    ex_np, ex_dev = host_experts(rng, E, H, I)
    idx = np.array([[1, 4, 1, 6], [2, 2, 2, 3], [7, -1, 9, 0]], dtype=np.int32)
    w = rng.random((T, k)).astype(np.float32)
    x32 = om.bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    x = torch.from_numpy(x32).to(DEV).to(torch.bfloat16)
    got = run(x, idx, w, ex_dev, I, validate=False)
    want = np.zeros((T, H))
    for t in range(T):
        seen = set()
        for j in range(k):
            e = int(idx[t, j])
            if 0 <= e < E and e not in seen:
                seen.add(e)
                want[t] += w[t, j] * omoe.expert_ffn(x32[t:t + 1], *ex_np[e])[0][0]
    rel = om.normwise_rel(got, want)
    print(f"duplicates / invalid ids: rel={rel:.3e}")
    assert rel <= TOL
    with pytest.raises(ValueError):
        run(x, idx, w, ex_dev, I, validate=True)
    # no valid id at all: zeros
    assert not run(x, np.full((T, k), 99, np.int32), w, ex_dev, I, validate=False).any()


def test_routed_decode_errors():
    from k3hip import _lib
    from k3hip.moe import moe_routed_decode
    rng = np.random.default_rng(3)
    _, ex_dev = host_experts(rng, 4, 256, 128)
    tab = table_of(ex_dev)
    x = torch.zeros(9, 256, dtype=torch.bfloat16, device=DEV)
    ids = torch.zeros(9, 2, dtype=torch.int64, device=DEV)
    wts = torch.ones(9, 2, device=DEV)
    with pytest.raises(ValueError, match="T=9"):
        moe_routed_decode(x, ids, wts, tab, 128)
    with pytest.raises(ValueError, match="multiple of 128"):
        moe_routed_decode(x[:4, :200], ids[:4], wts[:4], tab, 128)
    ws = torch.zeros(16, dtype=torch.uint8, device=DEV)
    with pytest.raises(ValueError, match="workspace"):
        _lib.call("k3_moe_routed_decode", x.data_ptr(), _lib.K3_BF16, ids.int().data_ptr(), wts.data_ptr(),
                  tab.data_ptr(), x.data_ptr(), _lib.K3_F32, 2, 256, 128, 4, 2, _lib.K3_ACT_SILU, 1.0, 0.0,
                  ws.data_ptr(), ws.numel(), None)


def test_routed_moe_fp32_wide_rows():
    """fp32 hidden states too wide to stage in one batch (5 and 8 tokens x 4096 fp32: 80 and
    128 KB): the router rows and the shared (gate, up) pairs run the persistent row kernel,
    its plain set and its pair set, the shared down rows the batched one; against the fp64
    layer."""
    from k3hip.moe import MoEConfig, RoutedMoE
    H, I, E, k, Is = 4096, 256, 32, 4, 512
    rng = np.random.default_rng(97)
    ex_np, ex_dev = host_experts(rng, E, H, I)
    router_w = om.bf16_round((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    shared = tuple(om.bf16_round((rng.standard_normal(sh) * 0.02).astype(np.float32))
                   for sh in ((Is, H), (Is, H), (H, Is)))
    w = {"gate.weight": torch.from_numpy(router_w).to(DEV).to(torch.bfloat16)}
    for name, a in zip(("gate", "up", "down"), shared):
        w[f"shared_experts.{name}_proj.weight"] = torch.from_numpy(a).to(DEV).to(torch.bfloat16)
    cfg = MoEConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, num_experts_per_token=k,
                    shared_intermediate_size=Is, router="softmax", activation="silu")
    which = {"w1": 0, "w3": 1, "w2": 2}
    moe = RoutedMoE(cfg, 0, w, lambda L, e, wh: ex_dev[e][which[wh]])
    experts = {e: ex_np[e] for e in range(E)}
    for T in (5, 8):
        x32 = rng.standard_normal((T, H)).astype(np.float32)
        y, r = moe(torch.from_numpy(x32).to(DEV), return_router=True)
        idx, wts, _, _ = omoe.route_softmax(x32, router_w, k, True, 1.0)
        assert np.array_equal(np.sort(r.expert_indices.cpu().numpy(), -1), np.sort(idx, -1))
        want = omoe.moe_layer(x32, idx, wts, experts, shared, kind="silu")
        rel = om.normwise_rel(y.float().cpu().numpy(), want)
        print(f"fp32 x, T={T}, H={H}: rel={rel:.3e}")
        assert rel <= TOL, rel


@pytest.mark.parametrize("router,xdt,Is", [("softmax", torch.bfloat16, 512), ("sigmoid_bias", torch.float32, 0),
                                           ("sigmoid_bias", torch.bfloat16, 1024)])
def test_routed_moe_few_tokens_and_prefill_dispatch(router, xdt, Is):
    """RoutedMoE.__call__: one token runs the fused layer, 2..8 tokens the whole-layer
    multi-token decode (k3_moe_layer_decode_multi: router and shared rows on HIP, each
    selected expert read once), more the grouped prefill; each against the fp64 layer with
    its shared expert, the router records (ids, weights, raw and corrected scores) against
    the oracle's."""
    from k3hip.moe import MoEConfig, RoutedMoE
    H, I, E, k = 2048, 512, 64, 8
    rng = np.random.default_rng(91 + Is)
    ex_np, ex_dev = host_experts(rng, E, H, I)
    router_w = om.bf16_round((rng.standard_normal((E, H)) * 0.02).astype(np.float32))
    w = {"gate.weight": torch.from_numpy(router_w).to(DEV).to(torch.bfloat16)}
    bias = None
    if router == "sigmoid_bias":
        bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
        w["gate.e_score_correction_bias"] = torch.from_numpy(bias).to(DEV)
    shared = None
    if Is:
        shared = tuple(om.bf16_round((rng.standard_normal(s) * 0.02).astype(np.float32))
                       for s in ((Is, H), (Is, H), (H, Is)))
        for name, a in zip(("gate", "up", "down"), shared):
            w[f"shared_experts.{name}_proj.weight"] = torch.from_numpy(a).to(DEV).to(torch.bfloat16)
    act, beta, lbeta = ("situ", 2.0, 3.0) if router == "sigmoid_bias" else ("silu", 1.0, None)
    cfg = MoEConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, num_experts_per_token=k,
                    shared_intermediate_size=Is, router=router, activation=act, situ_beta=beta,
                    situ_linear_beta=lbeta, routed_scaling_factor=2.5 if bias is not None else 1.0)
    which = {"w1": 0, "w3": 1, "w2": 2}
    moe = RoutedMoE(cfg, 0, w, lambda L, e, wh: ex_dev[e][which[wh]])
    experts = {e: ex_np[e] for e in range(E)}
    for T, tol in ((1, TOL), (2, TOL), (4, TOL), (8, TOL), (12, 5e-4)):
        x32 = rng.standard_normal((T, H)).astype(np.float32)
        if xdt == torch.bfloat16:
            x32 = om.bf16_round(x32)
        y, r = moe(torch.from_numpy(x32).to(DEV).to(xdt), return_router=True)
        if bias is None:
            idx, wts, raw, _ = omoe.route_softmax(x32, router_w, k, True, 1.0)
            corr = raw
        else:
            idx, wts, raw, corr = omoe.route_sigmoid_bias(x32, router_w, bias, k, True, 2.5)
        assert np.array_equal(np.sort(r.expert_indices.cpu().numpy(), -1), np.sort(idx, -1))
        got_w = np.take_along_axis(r.expert_weights.cpu().numpy(), np.argsort(r.expert_indices.cpu().numpy(), -1), -1)
        assert np.allclose(got_w, np.take_along_axis(wts, np.argsort(idx, -1), -1), rtol=1e-5, atol=1e-7)
        assert np.allclose(r.raw_scores.cpu().numpy(), raw, rtol=1e-4, atol=1e-7)
        assert np.allclose(r.corrected_scores.cpu().numpy(), corr, rtol=1e-4, atol=1e-6)
        want = omoe.moe_layer(x32, idx, wts, experts, shared, kind=act, beta=beta, linear_beta=lbeta)
        rel = om.normwise_rel(y.cpu().numpy(), want)
        print(f"RoutedMoE {router} {xdt} Is={Is} T={T}: rel={rel:.3e}")
        assert rel <= tol, (T, rel)


def test_layer_decode_multi_repeatable_and_bf16_out():
    """The whole-layer multi-token entry point twice on one workspace (every record it reads
    rewritten by the call itself): bit-identical; bf16 output is the fp32 output rounded."""
    from k3hip import _lib
    from k3hip import _torch as Tt
    from k3hip.moe import MoEConfig, RoutedMoE
    H, I, E, k, Is, T = 1024, 256, 32, 4, 256, 5
    rng = np.random.default_rng(5)
    ex_np, ex_dev = host_experts(rng, E, H, I)
    w = {"gate.weight": (torch.randn(E, H, device=DEV) * 0.02).to(torch.bfloat16)}
    for name, shape in (("gate", (Is, H)), ("up", (Is, H)), ("down", (H, Is))):
        w[f"shared_experts.{name}_proj.weight"] = (torch.randn(*shape, device=DEV) * 0.02).to(torch.bfloat16)
    cfg = MoEConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, num_experts_per_token=k,
                    shared_intermediate_size=Is)
    which = {"w1": 0, "w3": 1, "w2": 2}
    moe = RoutedMoE(cfg, 0, w, lambda L, e, wh: ex_dev[e][which[wh]])
    x = torch.randn(T, H, device=DEV).to(torch.bfloat16)
    a, b = moe(x), moe(x)
    assert torch.equal(a, b)
    c = moe(x, out_dtype=torch.bfloat16)
    assert torch.equal(c, a.to(torch.bfloat16))
    ws = torch.zeros(8, dtype=torch.uint8, device=DEV)
    out = torch.empty(T, H, device=DEV)
    with pytest.raises(ValueError, match="workspace"):
        _lib.call("k3_moe_layer_decode_multi", Tt.ptr(x), _lib.K3_BF16, Tt.ptr(moe.gate_w), None, 0, 1, 1.0,
                  Tt.ptr(moe.expert_table()), Tt.ptr(moe.sh_gate), Tt.ptr(moe.sh_up), Tt.ptr(moe.sh_down),
                  Tt.ptr(out), _lib.K3_F32, T, H, I, Is, E, k, 0, 1.0, 0.0, Tt.ptr(ws), ws.numel(), None)


@pytest.mark.parametrize("T", [4, 8])
def test_latent_moe_few_tokens_k3_shapes(T):
    """K3's routed layer (latent 3584, experts [3072 x 3584], top-16 of 896 distinct experts
    on the device, shared width 6144) for four and eight decode tokens through the
    multi-token path (eight tokens x top-16: the 128 (token, slot) pairs the union holds at
    most, and the fp32 act rows the persistent row form stages), against the fp64 oracle with
    the bf16 latent state."""
    from test_gpu_latent_moe import K3_CFG, K3Cfg, check
    check(K3Cfg(**K3_CFG), seed=52 + T, T=T, on_device=True)


def test_layers_without_side_stream():
    """Both whole-layer multi-token entry points with the side stream switched off
    (K3HIP_SIDE_STREAM=0, read once per process, so in a child process): the 384-expert
    layer then takes the shared gate/up rows in R and the shared down rows as extra blocks of
    D's launch, the latent layer the shared rows in order on the caller's stream; both
    against the fp64 oracle, as with the side stream."""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    code = ("import sys, torch; sys.path[:0] = [{t!r}, {r!r}, {p!r}]\n"
            "from test_gpu_moe_multi import test_routed_moe_few_tokens_and_prefill_dispatch as f\n"
            "f('sigmoid_bias', torch.bfloat16, 1024)\n"
            "from test_gpu_latent_moe import K3Cfg, check\n"
            "check(K3Cfg(hidden_size=1024, routed_expert_hidden_size=512, moe_intermediate_size=256, num_experts=16,"
            " num_experts_per_token=4), seed=90, T=4)\n"
            "print('side stream off: ok')\n").format(t=str(root / "tests"), r=str(root),
                                                     p=str(root / "kimi-k3-mlx-macmini_amd"))
    env = dict(os.environ, K3HIP_SIDE_STREAM="0")
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:])
    assert res.returncode == 0 and "side stream off: ok" in res.stdout


def test_layers_first_call_under_capture():
    """A first call made while the caller's stream is capturing cannot create the side
    stream (stream and event creation are not capturable), so it runs the shared expert on
    the caller's stream inside the graph: in a child process whose first multi-token layer
    calls are captured (after one-token calls that build the expert tables), the replays
    equal the eager calls made afterwards (which create and use the side stream) bit for bit,
    for both whole-layer multi-token entry points."""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    code = ("import sys, torch; sys.path[:0] = [{t!r}, {r!r}, {p!r}]\n"
            "from test_gpu_moe_multi import host_experts\n"
            "from test_gpu_latent_moe import K3Cfg, make\n"
            "from k3hip.moe import LatentMoE, MoEConfig, RoutedMoE\n"
            "import numpy as np\n"
            "dev = 'cuda'\n"
            "rng = np.random.default_rng(7)\n"
            "H, I, E, k, Is = 1024, 256, 16, 4, 512\n"
            "ex_np, ex_dev = host_experts(rng, E, H, I)\n"
            "w = {{'gate.weight': (torch.randn(E, H, device=dev) * 0.02).to(torch.bfloat16)}}\n"
            "for name, shape in (('gate', (Is, H)), ('up', (Is, H)), ('down', (H, Is))):\n"
            "    w['shared_experts.' + name + '_proj.weight'] = (torch.randn(*shape, device=dev) * 0.02).to(torch.bfloat16)\n"
            "which = {{'w1': 0, 'w3': 1, 'w2': 2}}\n"
            "moe = RoutedMoE(MoEConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, num_experts_per_token=k,"
            " shared_intermediate_size=Is), 0, w, lambda L, e, wh: ex_dev[e][which[wh]])\n"
            "cfg = K3Cfg(hidden_size=1024, routed_expert_hidden_size=512, moe_intermediate_size=256, num_experts=16,"
            " num_experts_per_token=4)\n"
            "wl, src, _ = make(91, 1024, 512, 256, 16, 4, 512)\n"
            "lat = LatentMoE(cfg, 0, wl, src)\n"
            "x = torch.randn(4, 1024, device=dev).to(torch.bfloat16)\n"
            "moe(x[:1]); lat(x[:1]); torch.cuda.synchronize()  # one-token calls: tables built, no side stream\n"
            "s = torch.cuda.Stream(); s.wait_stream(torch.cuda.current_stream())\n"
            "g = torch.cuda.CUDAGraph()\n"
            "with torch.cuda.graph(g, stream=s):\n"
            "    a, b = moe(x), lat(x)\n"
            "for _ in range(3):\n"
            "    g.replay(); torch.cuda.synchronize()\n"
            "    ea, eb = moe(x), lat(x); torch.cuda.synchronize()\n"
            "    assert torch.equal(a, ea) and torch.equal(b, eb)\n"
            "print('first call under capture: ok')\n").format(t=str(root / "tests"), r=str(root),
                                                              p=str(root / "kimi-k3-mlx-macmini_amd"))
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:])
    assert res.returncode == 0 and "first call under capture: ok" in res.stdout


@pytest.mark.gpu
def test_layers_capture_beside_eager_calls():
    """Calls under capture use the device's capture side stream, which stays in the capture
    until it ends; eager calls keep to the other side stream.  In a child process, with the
    side streams created by eager calls: thread A captures both multi-token layers (the latent
    layer after thread B's calls, so it finds the capture side stream already in its own
    capture) while thread B, with A's capture open, makes the same calls eagerly on its own
    stream.  B's results and every replay of A's graph equal the eager results bit for bit.
    (A second capture open on the device at once, which runs the shared rows on its own
    stream, is not exercised: torch's capture set-up synchronises the device, which an open
    capture forbids.)"""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    code = ("import sys, threading, torch; sys.path[:0] = [{t!r}, {r!r}, {p!r}]\n"
            "from test_gpu_moe_multi import host_experts\n"
            "from test_gpu_latent_moe import K3Cfg, make\n"
            "from k3hip.moe import LatentMoE, MoEConfig, RoutedMoE\n"
            "import numpy as np\n"
            "dev = 'cuda'\n"
            "rng = np.random.default_rng(8)\n"
            "H, I, E, k, Is = 1024, 256, 16, 4, 512\n"
            "ex_np, ex_dev = host_experts(rng, E, H, I)\n"
            "w = {{'gate.weight': (torch.randn(E, H, device=dev) * 0.02).to(torch.bfloat16)}}\n"
            "for name, shape in (('gate', (Is, H)), ('up', (Is, H)), ('down', (H, Is))):\n"
            "    w['shared_experts.' + name + '_proj.weight'] = (torch.randn(*shape, device=dev) * 0.02).to(torch.bfloat16)\n"
            "which = {{'w1': 0, 'w3': 1, 'w2': 2}}\n"
            "moe = RoutedMoE(MoEConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, num_experts_per_token=k,"
            " shared_intermediate_size=Is), 0, w, lambda L, e, wh: ex_dev[e][which[wh]])\n"
            "cfg = K3Cfg(hidden_size=1024, routed_expert_hidden_size=512, moe_intermediate_size=256, num_experts=16,"
            " num_experts_per_token=4)\n"
            "wl, src, _ = make(92, 1024, 512, 256, 16, 4, 512)\n"
            "lat = LatentMoE(cfg, 0, wl, src)\n"
            "x = torch.randn(4, 1024, device=dev).to(torch.bfloat16)\n"
            "ea, eb = moe(x).clone(), lat(x).clone(); torch.cuda.synchronize()  # side streams created\n"
            "a_in, b_done = threading.Event(), threading.Event()\n"
            "out, errs = {{}}, []\n"
            "def run(name, fn):\n"
            "    try:\n"
            "        fn()\n"
            "    except BaseException as e:\n"
            "        errs.append((name, repr(e)))\n"
            "    finally:\n"
            "        (a_in if name == 'A' else b_done).set()\n"
            "def cap_a():\n"
            "    s = torch.cuda.Stream(); s.wait_stream(torch.cuda.current_stream()); g = torch.cuda.CUDAGraph()\n"
            "    with torch.cuda.graph(g, stream=s, capture_error_mode='thread_local'):\n"
            "        out['a'] = moe(x)\n"
            "        a_in.set(); b_done.wait(60)\n"
            "        out['la'] = lat(x)\n"
            "    out['ga'] = g\n"
            "def eager_b():\n"
            "    a_in.wait(60)\n"
            "    s = torch.cuda.Stream(); s.wait_stream(torch.cuda.current_stream())\n"
            "    with torch.cuda.stream(s):\n"
            "        out['b'], out['lb'] = moe(x), lat(x)\n"
            "    s.synchronize()\n"
            "ts = [threading.Thread(target=run, args=(n, f)) for n, f in (('A', cap_a), ('B', eager_b))]\n"
            "for t in ts: t.start()\n"
            "for t in ts: t.join(120)\n"
            "assert not errs, errs\n"
            "assert torch.equal(out['b'], ea) and torch.equal(out['lb'], eb), 'eager call beside the captures'\n"
            "for i in range(3):\n"
            "    out['ga'].replay(); torch.cuda.synchronize()\n"
            "    assert torch.equal(out['a'], ea) and torch.equal(out['la'], eb), ('graph A', i)\n"
            "    assert torch.equal(moe(x), ea) and torch.equal(lat(x), eb); torch.cuda.synchronize()\n"
            "print('captures beside eager calls: ok')\n").format(t=str(root / "tests"), r=str(root),
                                                                   p=str(root / "kimi-k3-mlx-macmini_amd"))
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:])
    assert res.returncode == 0 and "captures beside eager calls: ok" in res.stdout
