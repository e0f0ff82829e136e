"""The integration gate on a miniature Kimi-K3 (tests/test_synthetic_integration.py:104-184
restated): the built MoE, MLA and KDA layers stacked under a token embedding and an
argmax head, fed from a synthetic checkpoint through the checkpoint reader.

  * the fused path (HIP MXFP4 kernels: one latent-layer decode per token, experts resident
    or read through the checkpoint source), the unfused path (the reference's loop with
    dequantise-then-BLAS projections) and the fp64 oracle stack all produce the same greedy
    tokens;
  * with the unfused path reading each projection when it is used, one decode token loads
    exactly top_k x 3 x (MoE layers) expert projections (test_synthetic_integration.py:169-175).
"""
from __future__ import annotations

import numpy as np
import pytest

from _mini_k3 import NTOK, PROMPT, GpuModel, MiniCfg, OracleModel, build_checkpoint

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def mini(tmp_path_factory):
    d = tmp_path_factory.mktemp("mini_k3")
    return d, build_checkpoint(d)


def _source(d):
    from k3hip.checkpoint import TensorSource
    return TensorSource(ckpt=d, device="cuda:0")


def test_every_path_gives_the_same_greedy_tokens(mini):
    d, tensors = mini
    src = _source(d)
    runs = {
        "fused, resident experts": GpuModel(src, fused=True, resident=True).generate(PROMPT, NTOK),
        "fused, experts from the source": GpuModel(src, fused=True, resident=False).generate(PROMPT, NTOK),
        "unfused (reference loop)": GpuModel(src, fused=False).generate(PROMPT, NTOK),
        "fp64 oracle": OracleModel(tensors).generate(PROMPT, NTOK),
    }
    base = runs["fused, resident experts"]
    print(runs)
    for name, toks in runs.items():
        assert toks == base, f"{name}: {toks} != fused {base}"
    assert len(set(base)) > 1, f"degenerate stream {base}"


def test_logits_match_the_oracle_each_step(mini):
    """The fused stack's last-token logits against the fp64 oracle's at every step of the
    greedy run (the bf16 MLA cache and fp32 arithmetic bound the difference)."""
    d, tensors = mini
    m = GpuModel(_source(d), fused=True, resident=True)
    o = OracleModel(tensors)
    ids, nxt = list(PROMPT), list(PROMPT)
    m.reset()
    for _ in range(NTOK):
        got = m.forward(nxt).double().cpu().numpy()
        want = o.logits(ids)
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel < 2e-3, rel
        tok = int(np.argmax(want))
        ids.append(tok)
        nxt = [tok]


def test_expert_projections_per_token(mini):
    d, _ = mini
    src = _source(d)
    cfg = MiniCfg()
    m = GpuModel(src, cfg, fused=False)
    m.reset()
    src.experts_loaded = 0
    m.forward([PROMPT[0]])
    n_moe = cfg.num_hidden_layers - cfg.first_k_dense_replace
    want = cfg.num_experts_per_token * 3 * n_moe
    assert src.experts_loaded == want, (src.experts_loaded, want)
