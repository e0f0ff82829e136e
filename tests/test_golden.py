"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU tests: the oracle reproduces every fixture (bit-exact for decode, 1e-12 for the fp64
products), so a change to the oracle cannot drift silently.  GPU tests: the HIP path,
called through the C-ABI wrappers, matches the fixtures -- decode bit-exact, products
within the normwise max-relative bar of each kernel's own parity test (all under 1e-3).
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import mla as omla
from oracle import moe as omoe
from oracle import mxfp4 as om

GOLD = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLD / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bf(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def layer_experts(g):
    n = sum(1 for k in g if k.endswith("_gp"))
    return [((g[f"e{e}_gp"], g[f"e{e}_gs"]), (g[f"e{e}_up"], g[f"e{e}_us"]), (g[f"e{e}_dp"], g[f"e{e}_ds"]))
            for e in range(n)]


# ------------------------------------------------------------------ oracle vs fixtures (CPU)
def test_oracle_reproduces_decode_kats():
    g = load("mxfp4_kat")
    assert np.array_equal(om.decode_mxfp4(g["packed"], g["scales"]).view(np.uint32), g["want_bits"])
    got = om.decode_mxfp4(g["packed_s"], g["scales_s"])[:, 0]
    assert np.array_equal(got.view(np.uint32), g["want_s_bits"])


def test_oracle_reproduces_matvec():
    g = load("matvec_n128_k256")
    assert np.allclose(om.matvec_f64(g["x"], g["packed"], g["scales"]), g["want"], rtol=1e-12, atol=0)


def test_oracle_reproduces_expert():
    g = load("expert_h256_i128")
    x = bf(g["x_bf16"])
    pairs = (g["gp"], g["gs"]), (g["up"], g["us"]), (g["dp"], g["ds"])
    assert om.normwise_rel(omoe.expert_ffn(x, *pairs, "silu")[0], g["want_silu"]) < 1e-12
    assert om.normwise_rel(omoe.expert_ffn(x, *pairs, "situ", beta=2.0, linear_beta=3.0)[0], g["want_situ"]) < 1e-12


def test_oracle_reproduces_layer():
    g = load("moe_layer_h128")
    x = bf(g["x_bf16"]).astype(np.float64)
    idx, w, probs, _ = omoe.route_softmax(x, bf(g["router_bf16"]), g["want_idx"].shape[1])
    assert np.array_equal(idx, g["want_idx"])
    assert np.allclose(w, g["want_w"], rtol=1e-12)
    shared = tuple(bf(g[f"sh_{n}_bf16"]) for n in ("gate", "up", "down"))
    y = omoe.moe_layer(x, idx, w, layer_experts(g), shared=shared)
    assert om.normwise_rel(y, g["want"]) < 1e-12


def test_oracle_reproduces_mla():
    g = load("mla_h2_t24")
    args = [bf(g[f"{k}_bf16"]) for k in ("q_nope", "q_rot", "w_uk", "w_uv", "lat", "rot")]
    assert om.normwise_rel(omla.mla_decode_absorbed(*args, 192 ** -0.5)[0], g["want"]) < 1e-12


# ------------------------------------------------------------------ HIP path vs fixtures (GPU)
def _t(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
    return t if dtype is None else t.to(dtype)


def _bf16(bits):
    import torch
    return _t(np.asarray(bits, np.uint16).view(np.int16)).view(torch.bfloat16)


@pytest.mark.gpu
def test_gpu_decode_kats_bit_exact():
    import torch
    from k3hip.mxfp4 import decode_mxfp4
    g = load("mxfp4_kat")
    got = decode_mxfp4(_t(g["packed"]), _t(g["scales"])).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), g["want_bits"])
    got_s = decode_mxfp4(_t(g["packed_s"]), _t(g["scales_s"])).cpu().numpy()[:, 0]
    assert np.array_equal(got_s.view(np.uint32), g["want_s_bits"])
    # bf16 output: every KAT value is bf16-exact
    got_b = decode_mxfp4(_t(g["packed"]), _t(g["scales"]), out_dtype=torch.bfloat16).float().cpu().numpy()
    assert np.array_equal(got_b.view(np.uint32), g["want_bits"])


@pytest.mark.gpu
def test_gpu_matvec_reference_gate():
    """tests/test_mxfp4_kernel.py:42-54: rel < 1e-6 against fp64, for M = 1, 2, 4."""
    from k3hip.mxfp4_matvec import mxfp4_matvec_fused
    g = load("matvec_n128_k256")
    for m in (1, 2, 4):
        got = mxfp4_matvec_fused(_t(g["x"][:m]), _t(g["packed"]), _t(g["scales"])).cpu().numpy()
        rel = om.normwise_rel(got, g["want"][:m])
        assert rel < 1e-6, (m, rel)


@pytest.mark.gpu
def test_gpu_expert_matches_fixture():
    from k3hip.moe import expert_ffn_fused
    g = load("expert_h256_i128")
    pairs = [(_t(g[p]), _t(g[s])) for p, s in (("gp", "gs"), ("up", "us"), ("dp", "ds"))]
    x = _bf16(g["x_bf16"])
    got = expert_ffn_fused(x, *pairs, act="silu").cpu().numpy()
    assert om.normwise_rel(got, g["want_silu"]) < 1e-5
    got = expert_ffn_fused(x, *pairs, act="situ", beta=2.0, linear_beta=3.0).cpu().numpy()
    assert om.normwise_rel(got, g["want_situ"]) < 1e-5


@pytest.mark.gpu
def test_gpu_layer_matches_fixture():
    from k3hip.moe import MoEConfig, RoutedMoE
    g = load("moe_layer_h128")
    experts = [tuple((_t(p), _t(s)) for p, s in ex) for ex in layer_experts(g)]
    E, H = g["router_bf16"].shape
    k = g["want_idx"].shape[1]
    Is = g["sh_gate_bf16"].shape[0]
    w = {"gate.weight": _bf16(g["router_bf16"]),
         "shared_experts.gate_proj.weight": _bf16(g["sh_gate_bf16"]),
         "shared_experts.up_proj.weight": _bf16(g["sh_up_bf16"]),
         "shared_experts.down_proj.weight": _bf16(g["sh_down_bf16"])}
    which = {"w1": 0, "w3": 1, "w2": 2}
    cfg = MoEConfig(hidden_size=H, moe_intermediate_size=experts[0][0][0].shape[0], num_experts=E,
                    num_experts_per_token=k, shared_intermediate_size=Is)
    moe = RoutedMoE(cfg, 0, w, lambda L, e, wh: experts[e][which[wh]])
    y, r = moe(_bf16(g["x_bf16"]), return_router=True)
    assert np.array_equal(r.expert_indices.cpu().numpy(), g["want_idx"])
    assert np.allclose(r.expert_weights.cpu().numpy(), g["want_w"], rtol=1e-5, atol=1e-7)
    assert om.normwise_rel(y.cpu().numpy(), g["want"]) < 1e-4


@pytest.mark.gpu
def test_gpu_mla_matches_fixture():
    from k3hip.mla import mla_decode_absorbed
    g = load("mla_h2_t24")
    args = [_bf16(g[f"{k}_bf16"]) for k in ("q_nope", "q_rot", "w_uk", "w_uv", "lat", "rot")]
    got = mla_decode_absorbed(*args, 192 ** -0.5).float().cpu().numpy()
    assert om.normwise_rel(got, g["want"]) < 1e-4
