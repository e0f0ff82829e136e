"""GPU parity of the single-launch expert FFN against the fp64 oracle (k3ref semantics)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _expert(rng, H, I):
    return (om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, H, I))


def _dev(pair):
    return tuple(torch.from_numpy(a).to(DEV) for a in pair)


@pytest.mark.parametrize("H,I", [(7168, 2048), (3584, 3072), (1024, 256), (2048, 384), (4096, 1024)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_expert_ffn_matches_oracle(H, I, xdt):
    from k3hip.moe import expert_ffn_fused
    rng = np.random.default_rng(H + I)
    g, u, d = _expert(rng, H, I)
    x32 = rng.standard_normal((1, H)).astype(np.float32)
    if xdt == torch.bfloat16:
        x32 = om.bf16_round(x32)
    x = torch.from_numpy(x32).to(DEV).to(xdt)
    got = expert_ffn_fused(x, _dev(g), _dev(u), _dev(d)).cpu().numpy()
    want = omoe.expert_ffn(x32, g, u, d)[0]
    assert om.normwise_rel(got, want) < 1e-5


@pytest.mark.parametrize("beta,lbeta", [(4.0, 25.0), (2.0, None)])
def test_expert_ffn_situ(beta, lbeta):
    from k3hip.moe import expert_ffn_fused
    rng = np.random.default_rng(5)
    H, I = 3584, 3072
    g, u, d = _expert(rng, H, I)
    x32 = om.bf16_round((rng.standard_normal((1, H)) * 0.05).astype(np.float32))
    x = torch.from_numpy(x32).to(DEV).to(torch.bfloat16)
    got = expert_ffn_fused(x, _dev(g), _dev(u), _dev(d), act="situ", beta=beta,
                           linear_beta=lbeta).cpu().numpy()
    want = omoe.expert_ffn(x32, g, u, d, kind="situ", beta=beta, linear_beta=lbeta)[0]
    assert om.normwise_rel(got, want) < 1e-5


def test_expert_ffn_repeated_calls_and_bf16_out():
    """Back-to-back launches sharing one workspace (and graph replays of them, with eager
    work between the replays) give bit-identical results."""
    from k3hip.moe import expert_ffn_fused
    rng = np.random.default_rng(9)
    H, I = 7168, 2048
    experts = [tuple(_dev(p) for p in _expert(rng, H, I)) for _ in range(3)]
    x = torch.from_numpy(om.bf16_round(rng.standard_normal((1, H)).astype(np.float32))).to(DEV).to(torch.bfloat16)
    ref = [expert_ffn_fused(x, *e).clone() for e in experts]
    for rep in range(20):
        e = rep % 3
        assert torch.equal(expert_ffn_fused(x, *experts[e]), ref[e])
    b = expert_ffn_fused(x, *experts[0], out_dtype=torch.bfloat16)
    assert torch.equal(b, ref[0].to(torch.bfloat16))
    g = torch.cuda.CUDAGraph()
    outs = []
    with torch.cuda.graph(g):
        for e in range(3):
            outs.append(expert_ffn_fused(x, *experts[e]))
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        for e in range(3):
            assert torch.equal(outs[e], ref[e])
        assert torch.equal(expert_ffn_fused(x, *experts[1]), ref[1])   # eager call between replays
