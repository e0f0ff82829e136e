"""GPU parity of K3's routed layer with the latent wrapper (LatentMoE, moe.py:110-132)
against the fp64 oracle (``oracle.moe.latent_moe``).

The latent state h = x W_down^T is bf16 in the reference (its bf16 matmul, moe.py:117) and
here (the decode kernel rounds its fp32 row dots; the grouped path uses torch's bf16 GEMM),
and the oracle rounds it the same way; a 1-ulp difference in a
few elements of h (fp32 vs fp64 accumulation before the rounding) and the grouped MFMA
path's ~1e-4 error set the bar of the grouped path (T > 8): normwise max-relative 5e-4 (its
own bar), under the 1e-3 bar of the matvec gate; at K3 shapes with all 896 experts distinct
the grouped path reaches 6.6e-4 (the scaled MFMA sums each 128-element dot about 12 bits
below its largest product, and SiTU's act carries about 12 bits in three E4M3 terms), so
that case is held to the 1e-3 gate itself.  One token runs the fused decode kernels,
which round h as the oracle does and accumulate in fp32: 1e-5.  Two to eight tokens run the
multi-token decode (k3_moe_latent_layer_decode_multi, fp32 accumulation, 1e-7 on the routed
part alone), where more latent elements can land one bf16 ulp from the oracle's rounding: a
latent element whose fp32 sum falls on the other side of a bf16 rounding boundary than the
fp64 one moves that token's output by a few 1e-4 (observed 6.0e-5 at K3 shapes and four
tokens, 2.1e-4 for one of eight tokens, every other token within 1e-6): 5e-4, the grouped
path's bar.  The router result is compared exactly (ids) and to 1e-5 (weights).
"""
from __future__ import annotations

import os
from dataclasses import dataclass

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL_GROUPED = 5e-4
TOL_DECODE = 1e-5
TOL_MULTI = 5e-4
TOL_GATE = 1e-3   # the matvec gate (normwise max-relative, fp32-accumulated)


@dataclass
class K3Cfg:
    """The K3Config fields the layer reads (air_llm/models/kimi_k3/config.py:13-35)."""
    hidden_size: int
    routed_expert_hidden_size: int
    moe_intermediate_size: int
    num_experts: int
    num_experts_per_token: int
    moe_renormalize: bool = True
    routed_scaling_factor: float = 2.5
    situ_beta: float = 2.0
    situ_linear_beta: float | None = 3.0
    rms_norm_eps: float = 1e-5


class HostExperts:
    """experts[e] for the oracle: the device expert's (packed, scales) pairs copied to host
    memory on access, so only the experts the tokens select are ever copied."""

    def __init__(self, ex_dev):
        self.ex_dev = ex_dev

    def __getitem__(self, e):
        return tuple(tuple(a.cpu().numpy() for a in pair) for pair in self.ex_dev[e])


def device_experts(E, L, I, seed):
    """E distinct MXFP4 experts drawn on the device (scale bytes in [118, 130])."""
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)

    def mx(n, kk):
        return (torch.randint(0, 256, (n, kk // 2), dtype=torch.uint8, device=DEV, generator=g),
                torch.randint(118, 131, (n, kk // 32), dtype=torch.uint8, device=DEV, generator=g))

    return [(mx(I, L), mx(I, L), mx(L, I)) for _ in range(E)]


def make(seed, H, L, I, E, k, Is, distinct=None, on_device=False):
    """Weights of one layer.  ``distinct`` weight sets behind the E table rows (all E by
    default), drawn on the host; ``on_device`` draws all E experts distinct on the device
    instead (full-size tables) and hands the oracle a copy-on-access mapping."""
    rng = np.random.default_rng(seed)
    D = distinct or E
    if on_device:
        experts_dev = device_experts(E, L, I, seed)
    else:
        experts_np = [(om.random_mxfp4(rng, I, L), om.random_mxfp4(rng, I, L), om.random_mxfp4(rng, L, I))
                      for _ in range(D)]
        experts_dev = [tuple(tuple(torch.from_numpy(a).to(DEV) for a in pair) for pair in ex) for ex in experts_np]
    bf = lambda a: om.bf16_round(np.asarray(a, np.float32))  # noqa: E731
    router_w = bf(rng.standard_normal((E, H)) * 0.02)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    down = bf(rng.standard_normal((L, H)) * 0.02)
    up = bf(rng.standard_normal((H, L)) * 0.02)
    norm_w = (1.0 + 0.1 * rng.standard_normal(L)).astype(np.float32)
    shared = tuple(bf(rng.standard_normal(s) * 0.02) for s in ((Is, H), (Is, H), (H, Is)))
    t = lambda a, dt=torch.bfloat16: torch.from_numpy(np.ascontiguousarray(a)).to(DEV).to(dt)  # noqa: E731
    w = {"gate.weight": t(router_w), "gate.e_score_correction_bias": t(bias, torch.float32),
         "routed_expert_down_proj.weight": t(down), "routed_expert_up_proj.weight": t(up),
         "routed_expert_norm.weight": t(norm_w, torch.float32),
         "shared_experts.gate_proj.weight": t(shared[0]), "shared_experts.up_proj.weight": t(shared[1]),
         "shared_experts.down_proj.weight": t(shared[2])}
    which_ix = {"w1": 0, "w3": 1, "w2": 2}

    def source(layer, e, which):
        return experts_dev[e % D][which_ix[which]]

    oracle_experts = HostExperts(experts_dev) if on_device else {e: experts_np[e % D] for e in range(E)}
    oracle_args = (router_w, bias, down, up, norm_w, oracle_experts, shared)
    return w, source, oracle_args


def check(cfg, seed, T, distinct=None, on_device=False, tol=None):
    from k3hip.moe import LatentMoE
    w, source, (router_w, bias, down, up, norm_w, experts, shared) = make(
        seed, cfg.hidden_size, cfg.routed_expert_hidden_size, cfg.moe_intermediate_size, cfg.num_experts,
        cfg.num_experts_per_token, 2 * cfg.moe_intermediate_size, distinct, on_device)
    moe = LatentMoE(cfg, 0, w, source)
    rng = np.random.default_rng(seed + 1)
    x = om.bf16_round(rng.standard_normal((T, cfg.hidden_size)).astype(np.float32))
    y, r = moe(torch.from_numpy(x).to(DEV).to(torch.bfloat16), return_router=True)
    want, idx, wts = omoe.latent_moe(x, router_w, bias, down, up, norm_w, experts, shared,
                                     cfg.num_experts_per_token, cfg.moe_renormalize, cfg.routed_scaling_factor,
                                     cfg.situ_beta, cfg.situ_linear_beta, cfg.rms_norm_eps, h_bf16=True,
                                     workers=max(1, min(16, len(os.sched_getaffinity(0)))) if on_device else 1)
    assert np.array_equal(r.expert_indices.cpu().numpy(), idx)
    assert np.allclose(r.expert_weights.cpu().numpy(), wts, rtol=1e-5, atol=1e-7)
    rel = om.normwise_rel(y.float().cpu().numpy(), want)
    print(f"T={T} E={cfg.num_experts} k={cfg.num_experts_per_token} distinct experts used "
          f"{len(set(idx.ravel().tolist()))} rel={rel:.2e}")
    if tol is None:
        tol = TOL_DECODE if T == 1 else TOL_MULTI if T <= moe.DECODE_TOKENS else TOL_GROUPED
    per_tok = [om.normwise_rel(y.float().cpu().numpy()[t], want[t]) for t in range(T)]
    print("per-token rel: " + " ".join(f"{v:.1e}" for v in per_tok))
    assert rel <= tol, rel


@pytest.mark.parametrize("T", [1, 5, 12])
def test_latent_moe_small(T):
    """T = 1: the fused decode (k3_moe_latent_layer_decode); T = 5: the multi-token decode
    (k3_moe_latent_layer_decode_multi); T = 12: the grouped path."""
    check(K3Cfg(hidden_size=256, routed_expert_hidden_size=128, moe_intermediate_size=128, num_experts=16,
                num_experts_per_token=4), seed=40 + T, T=T)


@pytest.mark.parametrize("T", [5, 8])
def test_latent_moe_few_tokens_wide_rows(T):
    """Two to eight tokens with fp32 row inputs too wide to stage in one batch: the shared
    down rows (act [T, 4096] fp32: 80 / 128 KB) run the persistent row kernel, and the
    normalised up rows (the latent state [T, 3072] fp32: 60 / 96 KB) the batched kernel at
    T = 5 and the persistent one, normalising as it stages, at T = 8."""
    check(K3Cfg(hidden_size=1024, routed_expert_hidden_size=3072, moe_intermediate_size=2048, num_experts=16,
                num_experts_per_token=4), seed=60 + T, T=T)


@pytest.mark.parametrize("T", [3, 4])
def test_latent_moe_few_tokens_wide_hidden(T):
    """bf16 hidden states of width 7168 at three and four tokens (43 / 57 KB: two staged
    batches) feeding the router, latent down and shared gate/up rows together; the latent
    state (fp32 [T, 1024]) stages in one batch."""
    check(K3Cfg(hidden_size=7168, routed_expert_hidden_size=1024, moe_intermediate_size=512, num_experts=16,
                num_experts_per_token=4), seed=70 + T, T=T)


def test_latent_moe_multi_graph_replay_and_threads():
    """Four tokens through the multi-token latent layer, whose shared expert runs on the
    library's side stream (forked at the start of the call, joined before the up rows):
    repeated eager calls are bit-identical; a CUDA graph of three calls replays
    bit-identically four times with eager calls between the replays; two host threads, each
    on its own stream, calling the layer 20 times together get the eager results."""
    import threading

    from k3hip.moe import LatentMoE
    cfg = K3Cfg(hidden_size=1024, routed_expert_hidden_size=512, moe_intermediate_size=256, num_experts=16,
                num_experts_per_token=4)
    w, source, _ = make(80, 1024, 512, 256, 16, 4, 512)
    moe = LatentMoE(cfg, 0, w, source)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(81)
    xs = [torch.randn(4, 1024, device=DEV, generator=gen).to(torch.bfloat16) for _ in range(3)]
    ref = [moe(x).clone() for x in xs]
    for x, r in zip(xs, ref):
        assert torch.equal(moe(x), r)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = [moe(x) for x in xs]
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o, r)
        assert torch.equal(moe(xs[i % 3]), ref[i % 3])   # eager work between replays
    torch.cuda.synchronize()
    bad = []

    def worker(i):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            ys = [moe(xs[i]) for _ in range(20)]
        s.synchronize()
        bad.extend((i, j) for j, y in enumerate(ys) if not torch.equal(y, ref[i]))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not bad, bad


K3_CFG = dict(hidden_size=7168, routed_expert_hidden_size=3584, moe_intermediate_size=3072, num_experts=896,
              num_experts_per_token=16)


def test_latent_moe_k3_shapes_decode():
    """K3's routed layer shapes: hidden 7168, latent 3584, experts [3072 x 3584], top-16 of
    896, all 896 experts distinct (15.7 GB drawn on the device), two shared experts (one MLP
    of width 6144); one decode token."""
    check(K3Cfg(**K3_CFG), seed=50, T=1, on_device=True)


def test_latent_moe_k3_shapes_grouped():
    """The same K3 shapes with 16 tokens: more than DECODE_TOKENS, so the grouped path runs
    (batched routing, latent down GEMM, k3_moe_grouped_ffn over 896 distinct experts, norm,
    up and shared GEMMs); 256 (token, slot) pairs each reach their own expert's weights."""
    check(K3Cfg(**K3_CFG), seed=51, T=16, on_device=True, tol=TOL_GATE)


def test_latent_moe_rejects_wrong_projection_shapes():
    from k3hip.moe import LatentMoE
    cfg = K3Cfg(hidden_size=256, routed_expert_hidden_size=128, moe_intermediate_size=128, num_experts=8,
                num_experts_per_token=2)
    w, source, _ = make(3, 256, 128, 128, 8, 2, 256)
    w["routed_expert_up_proj.weight"] = w["routed_expert_up_proj.weight"][:, :64]
    with pytest.raises(ValueError):
        LatentMoE(cfg, 0, w, source)
