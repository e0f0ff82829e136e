"""Checkpoint ingestion onto the GPU: a synthetic K3 MoE layer written as two safetensors
shards with the reference's tensor names is loaded through page-locked staging and
asynchronous copies, and K3's routed layer run on it matches the fp64 oracle run on the
arrays that were written (the same bar as tests/test_gpu_latent_moe.py)."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


@dataclass
class Cfg:
    hidden_size: int = 256
    routed_expert_hidden_size: int = 128
    moe_intermediate_size: int = 128
    num_experts: int = 16
    num_experts_per_token: int = 4
    moe_renormalize: bool = True
    routed_scaling_factor: float = 2.5
    situ_beta: float = 2.0
    situ_linear_beta: float | None = 3.0
    rms_norm_eps: float = 1e-5


def test_ingested_layer_matches_oracle(tmp_path):
    import _synth_ckpt
    from k3hip.checkpoint import TensorSource
    from k3hip.moe import LatentMoE
    c, L = Cfg(), 7
    ref = _synth_ckpt.make_k3_checkpoint(tmp_path, 11, L, c.hidden_size, c.routed_expert_hidden_size,
                                         c.moe_intermediate_size, c.num_experts, 2 * c.moe_intermediate_size,
                                         gap_expert=5)
    src = TensorSource(ckpt=tmp_path, stage_bytes=1 << 16)   # small staging: every buffer is reused
    w = src.moe_weights(L)
    assert w["gate.weight"].dtype == torch.bfloat16 and w["gate.e_score_correction_bias"].dtype == torch.float32
    res = src.load_experts(L, c.num_experts)
    # the per-projection path returns the same bytes
    for e, j, wh in ((0, 0, "w1"), (5, 1, "w3"), (15, 2, "w2")):
        p, s = src.expert_source(L, e, wh)
        rp, rs = res.source(L, e, wh)
        assert torch.equal(p, rp) and torch.equal(s, rs)
        assert np.array_equal(p.cpu().numpy(), ref["experts"][e][j][0])
        assert np.array_equal(s.cpu().numpy(), ref["experts"][e][j][1])
    moe = LatentMoE(c, L, w, res.source)
    rng = np.random.default_rng(12)
    x = om.bf16_round(rng.standard_normal((3, c.hidden_size)).astype(np.float32))
    y = moe(torch.from_numpy(x).to(DEV).to(torch.bfloat16)).float().cpu().numpy()
    d = ref["dense"]
    want, _, _ = omoe.latent_moe(x, d["gate.weight"], d["gate.e_score_correction_bias"],
                                 d["routed_expert_down_proj.weight"], d["routed_expert_up_proj.weight"],
                                 d["routed_expert_norm.weight"], ref["experts"], ref["shared"],
                                 c.num_experts_per_token, c.moe_renormalize, c.routed_scaling_factor,
                                 c.situ_beta, c.situ_linear_beta, c.rms_norm_eps, h_bf16=True)
    rel = om.normwise_rel(y, want)
    print(f"ingested layer rel={rel:.2e}")
    assert rel <= 1e-5
    src.close()


def test_load_experts_rejects_unrepresentable_scale(tmp_path):
    import _synth_ckpt
    from k3hip.checkpoint import TensorSource
    _synth_ckpt.make_k3_checkpoint(tmp_path, 13, 2, 128, 64, 64, 4, 128, bad_scale=(3, "w2"))
    src = TensorSource(ckpt=tmp_path)
    with pytest.raises(ValueError, match=r"experts\.3\.w2"):
        src.load_experts(2, 4)
    with pytest.raises(ValueError, match="scale range"):
        src.expert_source(2, 3, "w2")
    p, _ = src.expert_source(2, 3, "w1")          # the other projections load
    assert p.shape == (64, 32)
