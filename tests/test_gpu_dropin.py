"""GPU parity of the drop-in surface around the fused kernels, against the fp64 oracle:

* the batched router selection (k3_moe_topk) and ``route`` on many tokens
  (``air_llm/models/kimi_k3/moe.py:65-76``);
* ``_proj`` fused and unfused (``moe.py:79-88``) against ``oracle.matvec_f64``;
* the reference's validation mode: fp32 dense weights with ``fused=False``
  (``loader.py:90-95``, ``run.py:75-78``), and ``fused=False`` with bf16 weights (runtime
  mode's unfused definition), against the oracle and against the fused path;
* fp32 hidden states through the fused latent decode and the grouped prefill (the latent
  state stays fp32, as the reference's bf16 x fp32 promotion gives);
* an fp32 MLA cache (the reference's default dtype, ``attention_mla.py:164``).

Tolerances (normwise max-relative error against fp64, ``max|got - want| / max|want|``):
fp32 paths with exact products 1e-5; the grouped MFMA path on fp32 inputs, whose x
terms keep about 12 bits, 1e-3 (expected near 2e-4); the unfused bf16 path, whose gate /
up projections come out of bf16 GEMMs rounded to bf16 as MLX's do, 5e-3 (the reference's
own single-expert bar, ``tests/test_moe_mlx.py:102-109``).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf(a):
    return om.bf16_round(np.asarray(a, np.float32))


def t(a, dt=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV).to(dt)


# ---------------------------------------------------------------------- router selection

def _topk_run(logits, bias, kind, k, renorm=True, scaling=1.0):
    from k3hip import _lib
    from k3hip import _torch as T
    n, E = logits.shape
    lg = t(logits)
    idx = torch.empty((n, k), dtype=torch.int32, device=DEV)
    w = torch.empty((n, k), device=DEV)
    sc = torch.empty((n, E), device=DEV)
    co = torch.empty((n, E), device=DEV)
    _lib.call("k3_moe_topk", T.ptr(lg), E, n, E, T.ptr(None if bias is None else t(bias)), kind, int(renorm),
              float(scaling), k, T.ptr(idx), T.ptr(w), T.ptr(sc), T.ptr(co), T.stream(lg))
    torch.cuda.synchronize()
    return idx.cpu().numpy(), w.cpu().numpy(), sc.cpu().numpy(), co.cpu().numpy()


def _oracle_select(logits, bias, kind, k, renorm=True, scaling=1.0):
    """Selection on given logits, restated in fp64 from moe.py:67-76 (softmax form for the
    benchmark router); ties to the lower index."""
    lg = np.asarray(logits, np.float64)
    if kind == "softmax":
        z = np.exp(lg - lg.max(axis=-1, keepdims=True))
        raw = z / z.sum(axis=-1, keepdims=True)
        corr = raw
    else:
        raw = omoe.sigmoid(lg)
        corr = raw + np.asarray(bias, np.float64)
    idx = omoe.topk_lowest_index(corr, k)
    w = np.take_along_axis(raw, idx, axis=-1)
    if renorm and k > 1:
        w = w / (w.sum(axis=-1, keepdims=True) + 1e-20)
    return idx, w * scaling, raw, corr


@pytest.mark.parametrize("n,E,k,kind", [(37, 384, 8, "softmax"), (5, 896, 16, "sigmoid_bias"),
                                        (64, 16, 4, "sigmoid_bias"), (3, 1024, 1, "softmax")])
def test_topk_batched_matches_oracle(n, E, k, kind):
    from k3hip import _lib
    rng = np.random.default_rng(300 + E)
    logits = (rng.standard_normal((n, E)) * 2).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32) if kind == "sigmoid_bias" else None
    code = _lib.K3_ROUTE_SOFTMAX if kind == "softmax" else _lib.K3_ROUTE_SIGMOID_BIAS
    idx, w, sc, co = _topk_run(logits, bias, code, k, scaling=2.5)
    widx, ww, wraw, wcorr = _oracle_select(logits, bias, kind, k, scaling=2.5)
    assert np.array_equal(idx, widx)
    assert np.allclose(w, ww, rtol=2e-6, atol=1e-9)
    assert np.allclose(sc, wraw, rtol=2e-6, atol=1e-12)
    assert np.allclose(co, wcorr, rtol=2e-6, atol=1e-7)   # raw + bias in fp32 may nearly cancel


def test_topk_ties_go_to_lower_index_and_empty_batch():
    from k3hip import _lib
    logits = np.zeros((2, 64), np.float32)
    logits[1, [5, 9, 40]] = 1.0           # three equal winners
    idx, w, _, _ = _topk_run(logits, None, _lib.K3_ROUTE_SOFTMAX, 4)
    assert idx[0].tolist() == [0, 1, 2, 3]
    assert idx[1].tolist() == [5, 9, 40, 0]
    assert np.allclose(w.sum(axis=1), 1.0, rtol=1e-6)
    # NaN scores rank as -inf (sigmoid keeps the other scores finite): 17 first, then the
    # lowest indices among the NaN ties
    nan_row = np.full((1, 64), np.nan, np.float32)
    nan_row[0, 17] = 0.5
    idx, _, _, _ = _topk_run(nan_row, np.zeros(64, np.float32), _lib.K3_ROUTE_SIGMOID_BIAS, 3)
    assert idx[0].tolist() == [17, 0, 1]
    # T = 0 is a no-op
    from k3hip import _torch as T
    z = torch.empty(0, device=DEV)
    _lib.call("k3_moe_topk", T.ptr(z), 64, 0, 64, None, 0, 1, 1.0, 4, T.ptr(z), T.ptr(z), T.ptr(z), T.ptr(z),
              T.stream(z))


@pytest.mark.parametrize("case", ["ties_across_groups", "clustered", "all_equal", "random_1024", "unsampled",
                                  "softmax_nan"])
def test_topk_every_selection_path(case):
    """Rows built to reach each path of the selection: a few candidates at or above the
    bound sampled from the experts (the largest key of every 16 experts; random rows), more
    than 64 of them (a ranking level before the last: 100 hot experts in the first two
    groups of 64, or all logits equal: 241 candidates), fewer samples than k (every key
    ranked: 100 experts, top-12), ties across groups and waves, and a NaN logit under
    softmax (every probability NaN: the k lowest indices, NaN weights and scores)."""
    from k3hip import _lib
    rng = np.random.default_rng(sum(map(ord, case)))
    bias = None
    kind, code = "softmax", _lib.K3_ROUTE_SOFTMAX
    if case == "ties_across_groups":
        E, k = 384, 8
        logits = np.zeros((3, E), np.float32)
        logits[0, [5, 100, 300, 301]] = 3.0
        logits[0, [200, 7]] = 2.5
        logits[1, [383, 64, 128, 0]] = 1.0          # ties in four groups, three waves
        logits[2] = np.repeat(np.arange(6, dtype=np.float32), 64)[::-1].copy()  # group-constant
    elif case == "clustered":
        E, k = 896, 16
        kind, code = "sigmoid_bias", _lib.K3_ROUTE_SIGMOID_BIAS
        logits = rng.standard_normal((4, E)).astype(np.float32)
        logits[:, :100] += 4.0
        bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    elif case == "all_equal":
        E, k = 1024, 16
        logits = np.zeros((2, E), np.float32)
        logits[1, [1000, 999]] = 1.0
    elif case == "unsampled":
        E, k = 100, 12
        logits = (rng.standard_normal((4, E)) * 2).astype(np.float32)
        logits[3, ::7] = 5.0
    elif case == "random_1024":
        E, k = 1024, 16
        logits = (rng.standard_normal((8, E)) * 2).astype(np.float32)
    else:
        E, k = 384, 8
        logits = (rng.standard_normal((2, E)) * 2).astype(np.float32)
        logits[1, 200] = np.nan
    idx, w, sc, co = _topk_run(logits, bias, code, k, scaling=1.5)
    widx, ww, wraw, wcorr = _oracle_select(logits, bias, kind, k, scaling=1.5)
    assert np.array_equal(idx, widx)
    if case == "softmax_nan":
        assert np.allclose(w[0], ww[0], rtol=2e-6, atol=1e-9)
        assert idx[1].tolist() == list(range(k))
        assert np.isnan(w[1]).all() and np.isnan(sc[1]).all() and np.isnan(co[1]).all()
        return
    assert np.allclose(w, ww, rtol=2e-6, atol=1e-9)
    assert np.allclose(sc, wraw, rtol=2e-6, atol=1e-12)
    assert np.allclose(co, wcorr, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("E,k", [(384, 8), (896, 16), (1024, 16), (100, 12)])
def test_topk_many_rows_with_ties(E, k):
    """512 softmax rows whose logits lie on a half-integer grid, so most rows hold exact ties
    across 64-expert groups and across the sampled bound: the selection (order included)
    must be the oracle's, ties to the lower index."""
    from k3hip import _lib
    rng = np.random.default_rng(E * 31 + k)
    logits = (np.round(rng.standard_normal((512, E)) * 3.0) / 2.0).astype(np.float32)
    idx, w, sc, _ = _topk_run(logits, None, _lib.K3_ROUTE_SOFTMAX, k, scaling=1.0)
    widx, ww, wraw, _ = _oracle_select(logits, None, "softmax", k)
    assert np.array_equal(idx, widx)
    assert np.allclose(w, ww, rtol=2e-6, atol=1e-9)
    assert np.allclose(sc, wraw, rtol=2e-6, atol=1e-12)


def test_topk_rejects_bad_arguments():
    from k3hip import _lib
    from k3hip import _torch as T
    z = torch.zeros(64, device=DEV)
    with pytest.raises(ValueError):   # top_k > 16
        _lib.call("k3_moe_topk", T.ptr(z), 64, 1, 64, None, 0, 1, 1.0, 17, T.ptr(z), T.ptr(z), T.ptr(z), T.ptr(z),
                  T.stream(z))
    with pytest.raises(ValueError):   # row stride below E
        _lib.call("k3_moe_topk", T.ptr(z), 32, 1, 64, None, 0, 1, 1.0, 4, T.ptr(z), T.ptr(z), T.ptr(z), T.ptr(z),
                  T.stream(z))


# ---------------------------------------------------------------------- K3 latent layer

@dataclass
class K3Cfg:
    """The K3Config fields the layer reads (air_llm/models/kimi_k3/config.py:13-35)."""
    hidden_size: int = 512
    routed_expert_hidden_size: int = 256
    moe_intermediate_size: int = 256
    num_experts: int = 24
    num_experts_per_token: int = 6
    moe_renormalize: bool = True
    routed_scaling_factor: float = 2.5
    situ_beta: float = 2.0
    situ_linear_beta: float | None = 3.0
    rms_norm_eps: float = 1e-5


def make_latent(seed, cfg, dense_dtype=torch.bfloat16):
    """Random K3-style layer: dense weights bf16-exact values stored as dense_dtype (the
    validation loader's fp32 copies hold the same numbers)."""
    H, L, I, E = cfg.hidden_size, cfg.routed_expert_hidden_size, cfg.moe_intermediate_size, cfg.num_experts
    Is = 2 * I
    rng = np.random.default_rng(seed)
    experts_np = [(om.random_mxfp4(rng, I, L), om.random_mxfp4(rng, I, L), om.random_mxfp4(rng, L, I))
                  for _ in range(E)]
    experts_dev = [tuple(tuple(torch.from_numpy(a).to(DEV) for a in pair) for pair in ex) for ex in experts_np]
    router_w = bf(rng.standard_normal((E, H)) * 0.05)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32)
    down = bf(rng.standard_normal((L, H)) * 0.05)
    up = bf(rng.standard_normal((H, L)) * 0.05)
    norm_w = (1.0 + 0.1 * rng.standard_normal(L)).astype(np.float32)
    shared = tuple(bf(rng.standard_normal(s) * 0.05) for s in ((Is, H), (Is, H), (H, Is)))
    w = {"gate.weight": t(router_w, dense_dtype), "gate.e_score_correction_bias": t(bias),
         "routed_expert_down_proj.weight": t(down, dense_dtype), "routed_expert_up_proj.weight": t(up, dense_dtype),
         "routed_expert_norm.weight": t(norm_w),
         "shared_experts.gate_proj.weight": t(shared[0], dense_dtype),
         "shared_experts.up_proj.weight": t(shared[1], dense_dtype),
         "shared_experts.down_proj.weight": t(shared[2], dense_dtype)}
    which_ix = {"w1": 0, "w3": 1, "w2": 2}

    def source(layer, e, which):
        return experts_dev[e][which_ix[which]]

    oracle_args = (router_w, bias, down, up, norm_w, dict(enumerate(experts_np)), shared)
    return w, source, oracle_args


def oracle_latent(cfg, x, args, h_bf16):
    router_w, bias, down, up, norm_w, experts, shared = args
    return omoe.latent_moe(x, router_w, bias, down, up, norm_w, experts, shared, cfg.num_experts_per_token,
                           cfg.moe_renormalize, cfg.routed_scaling_factor, cfg.situ_beta, cfg.situ_linear_beta,
                           cfg.rms_norm_eps, h_bf16=h_bf16)


def test_proj_fused_and_unfused_match_oracle_matvec():
    """_proj(h, e, which) for every projection: the fused MXFP4 matvec and the unfused
    decode-then-matmul against oracle.matvec_f64 on the bit-exact decoded weights."""
    from k3hip.moe import LatentMoE
    cfg = K3Cfg()
    w, source, args = make_latent(61, cfg)
    experts = args[5]
    rng = np.random.default_rng(62)
    for fused in (True, False):
        moe = LatentMoE(cfg, 0, w, source, fused=fused)
        for which, width in (("w1", cfg.routed_expert_hidden_size), ("w3", cfg.routed_expert_hidden_size),
                             ("w2", cfg.moe_intermediate_size)):
            h = rng.standard_normal((3, width)).astype(np.float32)
            got = moe._proj(t(h), 7, which).float().cpu().numpy()
            want = om.matvec_f64(h, *experts[7][{"w1": 0, "w3": 1, "w2": 2}[which]])
            rel = om.normwise_rel(got, want)
            assert rel <= 1e-5, (fused, which, rel)


def test_latent_moe_validation_mode_fp32_weights_unfused():
    """The reference's validation mode: fp32 dense weights, fused=False, fp32 hidden states
    that are not bf16 values.  Every projection is exact-product fp32 (the MXFP4 weights
    decode exactly to bf16, h stays fp32), so the result tracks the fp64 oracle with the
    unrounded latent state to fp32 accuracy."""
    from k3hip.moe import LatentMoE
    cfg = K3Cfg()
    w, source, args = make_latent(63, cfg, dense_dtype=torch.float32)
    moe = LatentMoE(cfg, 0, w, source, fused=False)
    assert not moe._fast
    x = np.random.default_rng(64).standard_normal((5, cfg.hidden_size)).astype(np.float32)
    y, r = moe(t(x), return_router=True)
    want, idx, wts = oracle_latent(cfg, x, args, h_bf16=False)
    assert np.array_equal(r.expert_indices.cpu().numpy(), idx)
    assert np.allclose(r.expert_weights.cpu().numpy(), wts, rtol=1e-5, atol=1e-7)
    rel = om.normwise_rel(y.cpu().numpy(), want)
    print(f"validation mode rel {rel:.2e}")
    assert rel <= 1e-5


def test_latent_moe_fp32_weights_fused_runs_reference_structure():
    """fp32 dense weights with fused=True: the dense projections stay fp32 on the BLAS
    library and the expert projections use the fused matvec."""
    from k3hip.moe import LatentMoE
    cfg = K3Cfg()
    w, source, args = make_latent(65, cfg, dense_dtype=torch.float32)
    moe = LatentMoE(cfg, 0, w, source, fused=True)
    x = np.random.default_rng(66).standard_normal((3, cfg.hidden_size)).astype(np.float32)
    want, _, _ = oracle_latent(cfg, x, args, h_bf16=False)
    assert om.normwise_rel(moe(t(x)).cpu().numpy(), want) <= 1e-5


def test_latent_moe_unfused_bf16_matches_fused():
    """Runtime mode with fused=False (bf16 weights and hidden states): the reference's
    unfused definition, whose bf16 GEMMs round gate / up to bf16, against the fused path and
    against the oracle (the reference's modes gate, tests/test_numerical_modes.py:52-73)."""
    from k3hip.moe import LatentMoE
    cfg = K3Cfg()
    w, source, args = make_latent(67, cfg)
    x = bf(np.random.default_rng(68).standard_normal((4, cfg.hidden_size)))
    xd = t(x, torch.bfloat16)
    fused = LatentMoE(cfg, 0, w, source, fused=True)(xd).cpu().numpy()
    unfused_moe = LatentMoE(cfg, 0, w, source, fused=False)
    y_unf, r = unfused_moe(xd, return_router=True)
    want, idx, _ = oracle_latent(cfg, x, args, h_bf16=True)
    assert np.array_equal(r.expert_indices.cpu().numpy(), idx)
    rel_f = om.normwise_rel(fused, want)
    rel_u = om.normwise_rel(y_unf.cpu().numpy(), want)
    rel_fu = om.normwise_rel(y_unf.cpu().numpy(), fused)
    print(f"fused {rel_f:.2e}  unfused {rel_u:.2e}  unfused vs fused {rel_fu:.2e}")
    assert rel_f <= 1e-5 and rel_u <= 5e-3 and rel_fu <= 5e-3


@pytest.mark.parametrize("T", [1, 3, 12])
def test_latent_moe_fp32_hidden_states(T):
    """fp32 x that is not bf16-exact: the decode kernel (T <= 8) routes on x and keeps the
    latent state in fp32; the grouped path (T = 12) routes on the unrounded x and feeds
    the fp32 latent state to the MFMA GEMM as three E4M3 terms."""
    from k3hip.moe import LatentMoE
    cfg = K3Cfg()
    w, source, args = make_latent(70 + T, cfg)
    moe = LatentMoE(cfg, 0, w, source)
    x = np.random.default_rng(80 + T).standard_normal((T, cfg.hidden_size)).astype(np.float32)
    y, r = moe(t(x), return_router=True)
    want, idx, wts = oracle_latent(cfg, x, args, h_bf16=False)
    assert np.array_equal(r.expert_indices.cpu().numpy(), idx)
    assert np.allclose(r.expert_weights.cpu().numpy(), wts, rtol=1e-5, atol=1e-7)
    rel = om.normwise_rel(y.cpu().numpy(), want)
    print(f"T={T} fp32 x rel {rel:.2e}")
    assert rel <= (1e-5 if T <= moe.DECODE_TOKENS else 1e-3)


def test_latent_moe_route_is_batched_and_matches_decode_records():
    """route() on many tokens (one GEMM + one selection launch) agrees with the records the
    fused decode kernel writes for each token."""
    from k3hip.moe import LatentMoE
    cfg = K3Cfg()
    w, source, args = make_latent(90, cfg)
    moe = LatentMoE(cfg, 0, w, source)
    x = bf(np.random.default_rng(91).standard_normal((6, cfg.hidden_size)))
    r = moe.route(t(x, torch.bfloat16))
    _, rd = moe(t(x, torch.bfloat16), return_router=True)
    assert torch.equal(r.expert_indices, rd.expert_indices)
    assert torch.allclose(r.expert_weights, rd.expert_weights, rtol=1e-5, atol=1e-7)
    assert torch.allclose(r.raw_scores, rd.raw_scores, rtol=1e-5, atol=1e-7)


# ---------------------------------------------------------------------- plain routed layer

def test_routed_moe_unfused_and_fp32_weights_match_oracle():
    """The benchmark's softmax layer with a shared expert, fused=False and fp32 dense
    weights: route, the host loop over routed experts with decode + BLAS projections, the
    shared expert; against oracle.moe_layer."""
    from k3hip.moe import MoEConfig, RoutedMoE
    H, I, E, k, Is = 512, 256, 32, 4, 256
    rng = np.random.default_rng(95)
    experts_np = [(om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, H, I))
                  for _ in range(E)]
    experts_dev = [tuple(tuple(torch.from_numpy(a).to(DEV) for a in pair) for pair in ex) for ex in experts_np]
    router_w = bf(rng.standard_normal((E, H)) * 0.05)
    shared = tuple(bf(rng.standard_normal(s) * 0.05) for s in ((Is, H), (Is, H), (H, Is)))
    w = {"gate.weight": t(router_w)}
    for name, a in zip(("gate", "up", "down"), shared):
        w[f"shared_experts.{name}_proj.weight"] = t(a)
    cfg = MoEConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E, num_experts_per_token=k,
                    shared_intermediate_size=Is)
    which_ix = {"w1": 0, "w3": 1, "w2": 2}
    moe = RoutedMoE(cfg, 0, w, lambda L, e, wh: experts_dev[e][which_ix[wh]], fused=False)
    x = rng.standard_normal((4, H)).astype(np.float32)
    y, r = moe(t(x), return_router=True)
    idx, wts, _, _ = omoe.route_softmax(x, router_w, k)
    want = omoe.moe_layer(x, idx, wts, dict(enumerate(experts_np)), shared)
    assert np.array_equal(r.expert_indices.cpu().numpy(), idx)
    rel = om.normwise_rel(y.cpu().numpy(), want)
    print(f"routed unfused fp32 rel {rel:.2e}")
    assert rel <= 1e-5


# ---------------------------------------------------------------------- MLA fp32 cache

@dataclass
class MlaCfg:
    hidden_size: int = 512
    num_attention_heads: int = 8
    q_lora_rank: int = 384
    kv_lora_rank: int = 512
    qk_nope_head_dim: int = 128
    qk_rope_head_dim: int = 64
    v_head_dim: int = 128
    rms_norm_eps: float = 1e-5
    mla_use_output_gate: bool = True
    mla_cache_dtype: torch.dtype = torch.float32

    @property
    def q_head_dim(self):
        return self.qk_nope_head_dim + self.qk_rope_head_dim


def test_mla_fp32_cache_decode_matches_expanded_oracle():
    """The reference's default fp32 cache: prefill, then single-token steps, each against the
    fp64 expanded one-shot layer (k3ref/layers.py:152-185) on the same input."""
    from oracle import mla as omla
    from k3hip.mla import MLAAttention
    cfg = MlaCfg()
    rng = np.random.default_rng(101)
    w32 = omla.random_mla_weights(rng, cfg)
    attn = MLAAttention(cfg, {k: t(v) for k, v in w32.items()})
    T, prefill = 12, 8
    x = (rng.standard_normal((1, T, cfg.hidden_size)) * 0.5).astype(np.float32)
    xd = t(x)
    out, cache = attn(xd[:, :prefill])
    steps = [out.cpu().numpy()]
    for s in range(prefill, T):
        o, cache = attn(xd[:, s:s + 1], cache=cache)
        steps.append(o.cpu().numpy())
    assert cache.latent.dtype == torch.float32 and cache.length == T
    got = np.concatenate(steps, axis=1)[0]
    want = omla.mla_layer_expanded(cfg, {k: v.astype(np.float64) for k, v in w32.items()}, x)[0]
    rel = om.normwise_rel(got, want)
    print(f"fp32 cache rel {rel:.2e}")
    assert rel <= 1e-5
