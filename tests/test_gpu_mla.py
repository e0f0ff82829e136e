"""GPU parity of the latent-MLA absorbed decode kernels against the fp64 oracle.

Tolerance: normwise max-relative error (max|got - want| / max|want|) <= 1e-3, the bar of
the matvec gate; the hi/lo-split MFMA path is expected near 1e-5.  Cache and weights are
bf16 (the benchmark's storage); the oracle reads the same bf16 values as float64.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import pytest
import torch

from oracle import mla as omla
from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-3


def bf(a):
    return om.bf16_round(np.asarray(a, np.float32))


def make(seed, H, T, nope=128, v=128, cap=None, wstd=0.02):
    rng = np.random.default_rng(seed)
    q_nope = bf(rng.standard_normal((H, nope)))
    q_rot = bf(rng.standard_normal((H, 64)))
    w_uk = bf(rng.standard_normal((H, nope, 512)) * wstd)
    w_uv = bf(rng.standard_normal((H, v, 512)) * wstd)
    lat = bf(rng.standard_normal((T, 512)))
    rot = bf(rng.standard_normal((T, 64)))
    return q_nope, q_rot, w_uk, w_uv, lat, rot


def to_dev(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV).to(dtype)


def run(q_nope, q_rot, w_uk, w_uv, lat, rot, scale, qdtype=torch.bfloat16, out_dtype=torch.float32, cap=None):
    from k3hip.mla import mla_decode_absorbed
    T = lat.shape[0]
    if cap:  # cache rows inside a larger backing buffer (capacity > length)
        lb = torch.zeros(cap, 512, dtype=torch.bfloat16, device=DEV)
        rb = torch.zeros(cap, 64, dtype=torch.bfloat16, device=DEV)
        lb[:T] = to_dev(lat)
        rb[:T] = to_dev(rot)
        ld, rd = lb[:T], rb[:T]
    else:
        ld, rd = to_dev(lat), to_dev(rot)
    out = mla_decode_absorbed(to_dev(q_nope, qdtype), to_dev(q_rot, qdtype), to_dev(w_uk), to_dev(w_uv), ld, rd,
                              scale, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("H,T", [(32, 1), (32, 5), (32, 31), (32, 32), (32, 33), (64, 100), (64, 257),
                                 (8, 48), (96, 777), (64, 4096), (16, 4321)])
def test_mla_decode_matches_oracle(H, T):
    args = make(1000 + H + T, H, T)
    scale = 192 ** -0.5
    got = run(*args, scale)
    want = omla.mla_decode_absorbed(*args, scale)[0]
    rel = om.normwise_rel(got, want)
    print(f"H={H} T={T} rel={rel:.3e}")
    assert rel <= TOL, rel
    assert rel <= 1e-4, f"hi/lo MFMA path should be near fp32: {rel:.3e}"


@pytest.mark.parametrize("nope,v", [(128, 72), (128, 256), (128, 1024), (64, 128), (256, 128), (64, 200)])
def test_mla_decode_other_head_dims(nope, v):
    """q_nope widths other than 128 (W_UK rows of 64 and 256) and v_head_dim other than 128:
    v not a multiple of 16 (72, 200), and v past the merge's first batch of 128 W_UV rows
    (256, 1024), which reloads W_UV in further batches."""
    H, T = 16, 300
    args = make(2000 + nope + v, H, T, nope=nope, v=v)
    scale = (nope + 64) ** -0.5
    got = run(*args, scale)
    want = omla.mla_decode_absorbed(*args, scale)[0]
    rel = om.normwise_rel(got, want)
    print(f"nope={nope} v={v} rel={rel:.3e}")
    assert got.shape == (H, v)
    assert rel <= 1e-4, rel


def test_mla_decode_full_size_config():
    """64 heads, 32768 cached tokens, kv_lora_rank 512 + rope 64, scale 1/sqrt(192)."""
    args = make(1005, 64, 32768)
    got = run(*args, 192 ** -0.5)
    want = omla.mla_decode_absorbed(*args, 192 ** -0.5)[0]
    rel = om.normwise_rel(got, want)
    print(f"full size rel={rel:.3e}")
    assert rel <= TOL
    assert rel <= 1e-4, f"hi/lo MFMA path should be near fp32: {rel:.3e}"


def make_f32(seed, H, T):
    """As make(), with an fp32 cache whose values are not bf16 values (N(0,1) in fp32)."""
    q_nope, q_rot, w_uk, w_uv, _, _ = make(seed, H, 1)
    rng = np.random.default_rng(seed + 1)
    lat = rng.standard_normal((T, 512)).astype(np.float32)
    rot = rng.standard_normal((T, 64)).astype(np.float32)
    return q_nope, q_rot, w_uk, w_uv, lat, rot


def run_f32(q_nope, q_rot, w_uk, w_uv, lat, rot, scale, cap=None, qdtype=torch.bfloat16):
    """The core on an fp32 cache (k3_mla_decode_absorbed_f32), optionally inside a larger
    backing buffer."""
    from k3hip.mla import mla_decode_absorbed
    T = lat.shape[0]
    if cap:
        lb = torch.zeros(cap, 512, dtype=torch.float32, device=DEV)
        rb = torch.zeros(cap, 64, dtype=torch.float32, device=DEV)
        lb[:T] = to_dev(lat, torch.float32)
        rb[:T] = to_dev(rot, torch.float32)
        ld, rd = lb[:T], rb[:T]
    else:
        ld, rd = to_dev(lat, torch.float32), to_dev(rot, torch.float32)
    out = mla_decode_absorbed(to_dev(q_nope, qdtype), to_dev(q_rot, qdtype), to_dev(w_uk), to_dev(w_uv), ld, rd,
                              scale)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("H,T", [(32, 1), (32, 17), (32, 33), (64, 257), (8, 48), (96, 777), (16, 4321)])
def test_mla_decode_f32_cache_matches_oracle(H, T):
    """The reference's default fp32 cache: rows split into hi/lo bf16 planes as they are
    staged, all four products kept: within 1e-5 of the fp64 oracle on the fp32 values."""
    args = make_f32(3000 + H + T, H, T)
    scale = 192 ** -0.5
    got = run_f32(*args, scale)
    want = omla.mla_decode_absorbed(*args, scale)[0]
    rel = om.normwise_rel(got, want)
    print(f"fp32 cache H={H} T={T} rel={rel:.3e}")
    assert rel <= 1e-5, rel


def test_mla_decode_f32_cache_full_size_strided_fp32_query():
    """64 heads over 32768 fp32 cache rows inside a larger backing buffer (capacity 33024,
    as MLACache grows), fp32 queries: within 1e-5 of fp64; the bf16 core on the bf16
    rounding of the same cache differs from it by the cache rounding only."""
    args = make_f32(3005, 64, 32768)
    scale = 192 ** -0.5
    got = run_f32(*args, scale, cap=33024, qdtype=torch.float32)
    q_nope, q_rot, w_uk, w_uv, lat, rot = args
    want = omla.mla_decode_absorbed(*args, scale)[0]
    rel = om.normwise_rel(got, want)
    print(f"fp32 cache full size rel={rel:.3e}")
    assert rel <= 1e-5, rel
    lat16, rot16 = bf(lat), bf(rot)
    got16 = run(q_nope, q_rot, w_uk, w_uv, lat16, rot16, scale, qdtype=torch.float32)
    want16 = omla.mla_decode_absorbed(q_nope, q_rot, w_uk, w_uv, lat16, rot16, scale)[0]
    assert om.normwise_rel(got16, want16) <= 1e-4
    assert om.normwise_rel(got, got16) > 10 * rel   # the fp32 rows did not go through bf16


def test_mla_decode_strided_cache_and_fp32_query_and_bf16_out():
    args = list(make(7, 64, 600))
    rng = np.random.default_rng(8)
    args[0] = rng.standard_normal(args[0].shape).astype(np.float32)   # fp32 queries (not bf16-exact)
    args[1] = rng.standard_normal(args[1].shape).astype(np.float32)
    want = omla.mla_decode_absorbed(*args, 0.07)[0]
    got = run(*args, 0.07, qdtype=torch.float32, cap=1024)
    assert om.normwise_rel(got, want) <= 1e-4
    got16 = run(*args, 0.07, qdtype=torch.float32, cap=1024, out_dtype=torch.bfloat16)
    assert np.array_equal(got16, om.bf16_round(got.astype(np.float32))) or om.normwise_rel(got16, want) <= 4e-3


def test_mla_decode_peaked_softmax():
    """Large scores (scale 1): the softmax concentrates on a few tokens; the running max
    must carry the rescaling exactly across tiles and splits."""
    args = make(9, 32, 3000, wstd=0.2)
    got = run(*args, 1.0)
    want = omla.mla_decode_absorbed(*args, 1.0)[0]
    assert om.normwise_rel(got, want) <= TOL


def test_mla_decode_rising_scores_move_the_reference():
    """Scores that climb by 80..170 (log2 units) every 96 tokens, for half of the heads:
    a later tile of a split exceeds the head's reference max by far more than the kernel's
    headroom, so the reference moves and the accumulators are rescaled (several times per
    split and tile class); the other heads fall instead.  The rope column 0 carries the
    ramp."""
    H, T = 64, 20000
    q_nope, q_rot, w_uk, w_uv, lat, rot = make(11, H, T)
    q_rot[:, 0] = np.linspace(-2.0, 2.0, H).astype(np.float32)
    rot[:, 0] = (800.0 * ((np.arange(T) // 96) % 4)).astype(np.float32)
    args = (q_nope, bf(q_rot), w_uk, w_uv, lat, bf(rot))
    scale = 192 ** -0.5
    got = run(*args, scale)
    want = omla.mla_decode_absorbed(*args, scale)[0]
    rel = om.normwise_rel(got, want)
    print(f"rising scores rel={rel:.3e}")
    assert rel <= 1e-4, rel


def test_mla_decode_is_deterministic():
    args = make(10, 64, 5000)
    a = run(*args, 0.1)
    b = run(*args, 0.1)
    assert np.array_equal(a, b)


def test_mla_decode_errors():
    from k3hip.mla import mla_decode_absorbed
    q = torch.zeros(32, 128, dtype=torch.bfloat16, device=DEV)
    qr = torch.zeros(32, 64, dtype=torch.bfloat16, device=DEV)
    wk = torch.zeros(32, 128, 512, dtype=torch.bfloat16, device=DEV)
    wv = torch.zeros(32, 128, 512, dtype=torch.bfloat16, device=DEV)
    lat = torch.zeros(10, 512, dtype=torch.bfloat16, device=DEV)
    rot = torch.zeros(10, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        mla_decode_absorbed(q, qr, wk, wv, lat[:0], rot[:0], 0.1)            # empty cache
    with pytest.raises(ValueError):
        mla_decode_absorbed(q, qr, wk, wv, lat, rot[:9], 0.1)                # T mismatch
    with pytest.raises(TypeError):
        mla_decode_absorbed(q, qr, wk, wv, lat.half(), rot.half(), 0.1)      # fp16 cache
    with pytest.raises(TypeError):
        mla_decode_absorbed(q, qr, wk, wv, lat.float(), rot, 0.1)            # mixed cache dtypes
    with pytest.raises(ValueError):
        mla_decode_absorbed(q, qr, wk[:, :, :256], wv[:, :, :256], lat[:, :256], rot, 0.1)  # r != 512


# ------------------------------------------------------------------ layer gates N1 / N2

@dataclass
class Cfg:
    hidden_size: int = 512
    num_attention_heads: int = 8
    q_lora_rank: int = 384
    kv_lora_rank: int = 512
    qk_nope_head_dim: int = 128
    qk_rope_head_dim: int = 64
    v_head_dim: int = 128
    rms_norm_eps: float = 1e-5
    mla_use_output_gate: bool = True
    mla_cache_dtype: torch.dtype = torch.bfloat16

    @property
    def q_head_dim(self):
        return self.qk_nope_head_dim + self.qk_rope_head_dim


def test_mla_layer_incremental_decode_matches_one_shot_oracle():
    """Gates N1/N2 (tests/test_mla_cache.py:229-255) restated: prefill, then decode token
    by token through the HIP core; every step's output must match the fp64 one-shot layer.
    The cache is bf16, so the oracle runs on the same bf16-rounded latents: its kv path is
    re-derived from the cache the module actually stored."""
    from k3hip.mla import MLAAttention
    cfg = Cfg()
    rng = np.random.default_rng(11)
    w32 = omla.random_mla_weights(rng, cfg)
    w32["kv_b_proj.weight"] = bf(w32["kv_b_proj.weight"])
    wdev = {k: torch.from_numpy(v).to(DEV) for k, v in w32.items()}
    attn = MLAAttention(cfg, wdev)
    T, prefill = 40, 33
    x = (rng.standard_normal((1, T, cfg.hidden_size)) * 0.5).astype(np.float32)
    xd = torch.from_numpy(x).to(DEV)
    out, cache = attn(xd[:, :prefill])
    steps = [out.cpu().numpy()]
    for t in range(prefill, T):
        o, cache = attn(xd[:, t:t + 1], cache=cache)
        steps.append(o.cpu().numpy())
    inc = np.concatenate(steps, axis=1)[0]
    assert cache.length == T
    # oracle on the stored (bf16) latents: rebuild the per-step expectation from the core
    lat = cache.latent[0, :T].float().cpu().numpy().astype(np.float64)
    rot = cache.rot[0, :T].float().cpu().numpy().astype(np.float64)
    w = {k: v.astype(np.float64) for k, v in w32.items()}
    nh, nope, klr, vhd = cfg.num_attention_heads, 128, 512, 128
    kb = w["kv_b_proj.weight"].reshape(nh, nope + vhd, klr)
    rms = lambda a, g: g * a / np.sqrt((a * a).mean(-1, keepdims=True) + cfg.rms_norm_eps)  # noqa: E731
    worst = 0.0
    for t in range(prefill, T):
        q = (rms(x[0, t].astype(np.float64) @ w["q_a_proj.weight"].T, w["q_a_layernorm.weight"])
             @ w["q_b_proj.weight"].T).reshape(nh, cfg.q_head_dim)
        o = omla.mla_decode_absorbed(q[:, :nope], q[:, nope:], kb[:, :nope], kb[:, nope:], lat[:t + 1],
                                     rot[:t + 1], cfg.q_head_dim ** -0.5)[0].reshape(-1)
        o = o / (1.0 + np.exp(-(x[0, t].astype(np.float64) @ w["g_proj.weight"].T)))
        want = o @ w["o_proj.weight"].T
        worst = max(worst, om.normwise_rel(inc[t], want))
    print(f"worst decode-step rel {worst:.3e}")
    assert worst <= TOL
    # and the fp64 expanded one-shot layer (fp32 latents) within the bf16 cache's rounding
    full = omla.mla_layer_expanded(cfg, w, x)[0]
    assert om.normwise_rel(inc[prefill:], full[prefill:]) <= 2e-2
    assert cache.bytes_per_token() == (512 + 64) * 2
    assert cache.nbytes_used() == T * (512 + 64) * 2


def test_mla_layer_fp32_cache_decode_runs_hip_core():
    """The reference's default fp32 cache with the checkpoint's bf16 kv_b: a decode token
    runs the HIP core on the fp32 rows (k3_mla_decode_absorbed_f32); prefill, then
    single-token steps, each against the fp64 expanded one-shot layer
    (k3ref/layers.py:152-185) within 1e-5."""
    from k3hip import mla as kmla
    cfg = Cfg(mla_cache_dtype=torch.float32)
    rng = np.random.default_rng(23)
    w32 = omla.random_mla_weights(rng, cfg)
    w32["kv_b_proj.weight"] = bf(w32["kv_b_proj.weight"])
    wdev = {k: torch.from_numpy(v).to(DEV) for k, v in w32.items()}
    wdev["kv_b_proj.weight"] = wdev["kv_b_proj.weight"].to(torch.bfloat16)
    attn = kmla.MLAAttention(cfg, wdev)
    calls = []
    core = kmla.mla_decode_absorbed

    def counting(*a, **k):
        calls.append(a[4].dtype)
        return core(*a, **k)

    kmla.mla_decode_absorbed = counting
    try:
        T, prefill = 300, 290
        x = (rng.standard_normal((1, T, cfg.hidden_size)) * 0.5).astype(np.float32)
        xd = torch.from_numpy(x).to(DEV)
        out, cache = attn(xd[:, :prefill])
        steps = [out.cpu().numpy()]
        for t in range(prefill, T):
            o, cache = attn(xd[:, t:t + 1], cache=cache)
            steps.append(o.cpu().numpy())
    finally:
        kmla.mla_decode_absorbed = core
    assert calls == [torch.float32] * (T - prefill)           # every decode step ran the fp32 core
    assert cache.latent.dtype == torch.float32 and cache.length == T and cache.capacity == 512
    got = np.concatenate(steps, axis=1)[0]
    want = omla.mla_layer_expanded(cfg, {k: v.astype(np.float64) for k, v in w32.items()}, x)[0]
    rel = om.normwise_rel(got[prefill:], want[prefill:])
    print(f"fp32 cache decode steps rel {rel:.2e}")
    assert rel <= 1e-5


def test_mla_fused_decode_step_matches_torch_step_and_oracle():
    """bf16 projection weights select k3_mla_step_decode for the decode steps (projections,
    norms, cache append, core, gate, o_proj in HIP).  Each step is checked against the same
    module with the torch projections around the HIP core, on a copy of the same cache, and
    against the fp64 restatement on the latents the fused step stored."""
    from k3hip.mla import MLACache, MLAAttention
    cfg = Cfg()
    rng = np.random.default_rng(17)
    w32 = {k: bf(v) for k, v in omla.random_mla_weights(rng, cfg).items()}
    wdev = {k: torch.from_numpy(v).to(DEV).to(torch.bfloat16) for k, v in w32.items()}
    wdev["q_a_layernorm.weight"] = torch.from_numpy(w32["q_a_layernorm.weight"]).to(DEV)
    wdev["kv_a_layernorm.weight"] = torch.from_numpy(w32["kv_a_layernorm.weight"]).to(DEV)
    fused, ref = MLAAttention(cfg, wdev), MLAAttention(cfg, wdev)
    assert fused.fused_step
    ref.fused_step = False
    T, prefill = 262, 250                      # the decode steps cross the 256-row capacity step
    x = (rng.standard_normal((1, T, cfg.hidden_size)) * 0.5).astype(np.float32)
    xd = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    _, cache = fused(xd[:, :prefill])
    cref = MLACache(cache.latent.clone(), cache.rot.clone(), cache.length)
    w = {k: v.astype(np.float64) for k, v in w32.items()}
    nh, nope, klr, vhd = cfg.num_attention_heads, 128, 512, 128
    kb = w["kv_b_proj.weight"].reshape(nh, nope + vhd, klr)
    rms = lambda a, g: g * a / np.sqrt((a * a).mean(-1, keepdims=True) + cfg.rms_norm_eps)  # noqa: E731
    xb = om.bf16_round(x[0]).astype(np.float64)
    worst_ref = worst_oracle = 0.0
    for t in range(prefill, T):
        o, cache = fused(xd[:, t:t + 1], cache=cache)
        o_ref, cref = ref(xd[:, t:t + 1], cache=cref)
        assert cache.length == cref.length == t + 1
        got = o.float().cpu().numpy().reshape(-1)
        worst_ref = max(worst_ref, om.normwise_rel(got, o_ref.float().cpu().numpy().reshape(-1)))
        d = (cache.latent[0, t].float() - cref.latent[0, t].float()).abs().max().item()
        assert d <= 2 ** -7 * cref.latent[0, t].float().abs().max().item()       # one bf16 ulp at most
        assert torch.equal(cache.rot[0, t], cref.rot[0, t]) or \
            (cache.rot[0, t].float() - cref.rot[0, t].float()).abs().max().item() <= \
            2 ** -7 * cref.rot[0, t].float().abs().max().item()
        lat = cache.latent[0, :t + 1].float().cpu().numpy().astype(np.float64)
        rot = cache.rot[0, :t + 1].float().cpu().numpy().astype(np.float64)
        # the new cache row against fp64 directly: bf16(rmsnorm(kv_a x)) and bf16(rope part)
        ckv = xb[t] @ w["kv_a_proj_with_mqa.weight"].T
        lat_want = rms(ckv[:klr], w["kv_a_layernorm.weight"])
        assert np.abs(lat[t] - lat_want).max() <= 2 ** -8 * np.abs(lat_want).max()   # one bf16 rounding
        assert np.abs(rot[t] - ckv[klr:]).max() <= 2 ** -8 * np.abs(ckv[klr:]).max()
        q = (rms(xb[t] @ w["q_a_proj.weight"].T, w["q_a_layernorm.weight"]) @ w["q_b_proj.weight"].T
             ).reshape(nh, cfg.q_head_dim)
        oo = omla.mla_decode_absorbed(q[:, :nope], q[:, nope:], kb[:, :nope], kb[:, nope:], lat, rot,
                                      cfg.q_head_dim ** -0.5)[0].reshape(-1)
        oo = oo / (1.0 + np.exp(-(xb[t] @ w["g_proj.weight"].T)))
        worst_oracle = max(worst_oracle, om.normwise_rel(got, oo @ w["o_proj.weight"].T))
    print(f"fused step vs torch step {worst_ref:.2e}, vs oracle {worst_oracle:.2e}")
    assert worst_ref <= 1e-4 and worst_oracle <= 1e-4
    assert cache.capacity == 512


def test_mla_fused_decode_step_errors():
    from k3hip import _lib
    from k3hip.mla import MLAAttention
    cfg = Cfg()
    rng = np.random.default_rng(3)
    wdev = {k: torch.from_numpy(v).to(DEV).to(torch.bfloat16) for k, v in omla.random_mla_weights(rng, cfg).items()}
    attn = MLAAttention(cfg, wdev)
    x = torch.randn(1, 1, cfg.hidden_size, device=DEV).to(torch.bfloat16)
    o, cache = attn(x)                                  # no cache: a new one, position 0
    assert cache.length == 1 and torch.isfinite(o).all()
    lat, rot = cache.latent[0], cache.rot[0]
    out = torch.empty(cfg.hidden_size, device=DEV)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=DEV)
    with pytest.raises(ValueError, match="outside the cache"):
        _lib.call("k3_mla_step_decode", x.data_ptr(), _lib.K3_BF16, wdev["q_a_proj.weight"].data_ptr(),
                  attn._q_an32.data_ptr(), wdev["q_b_proj.weight"].data_ptr(),
                  wdev["kv_a_proj_with_mqa.weight"].data_ptr(), attn._kv_an32.data_ptr(), attn.wk.data_ptr(),
                  attn.wv.data_ptr(), None, wdev["o_proj.weight"].data_ptr(), lat.data_ptr(), 512, rot.data_ptr(),
                  64, cache.capacity, cache.capacity, 1e-5, 0.1, out.data_ptr(), _lib.K3_F32, cfg.hidden_size,
                  cfg.q_lora_rank, cfg.num_attention_heads, 128, 64, 128, 512, ws.data_ptr(), ws.numel(), None)


def test_mla_fused_decode_step_fp32_input_and_bf16_output():
    """The C-ABI step with fp32 x and bf16 out matches the bf16-x / fp32-out step on the
    same (bf16-representable) input to bf16 output rounding."""
    from k3hip import _lib
    from k3hip.mla import MLAAttention, new_cache
    cfg = Cfg()
    rng = np.random.default_rng(5)
    wdev = {k: torch.from_numpy(bf(v)).to(DEV).to(torch.bfloat16) for k, v in omla.random_mla_weights(rng, cfg).items()}
    attn = MLAAttention(cfg, wdev)
    x32 = torch.from_numpy(bf(rng.standard_normal(cfg.hidden_size) * 0.5)).to(DEV)
    outs = []
    for xin, odt in ((x32.to(torch.bfloat16), _lib.K3_F32), (x32, _lib.K3_BF16)):
        cache = new_cache(1, 512, 64, 1, torch.bfloat16, DEV)
        out = torch.empty(cfg.hidden_size, dtype=torch.float32 if odt == _lib.K3_F32 else torch.bfloat16, device=DEV)
        ws = torch.empty(1 << 22, dtype=torch.uint8, device=DEV)
        m = attn._mats
        _lib.call("k3_mla_step_decode", xin.data_ptr(), _lib.K3_BF16 if xin.dtype == torch.bfloat16 else _lib.K3_F32,
                  m["q_a"].data_ptr(), attn._q_an32.data_ptr(), m["q_b"].data_ptr(), m["kv_a"].data_ptr(),
                  attn._kv_an32.data_ptr(), attn.wk.data_ptr(), attn.wv.data_ptr(), m["g"].data_ptr(),
                  m["o"].data_ptr(), cache.latent.data_ptr(), 512, cache.rot.data_ptr(), 64, cache.capacity, 0,
                  1e-5, cfg.q_head_dim ** -0.5, out.data_ptr(), odt, cfg.hidden_size, cfg.q_lora_rank,
                  cfg.num_attention_heads, 128, 64, 128, 512, ws.data_ptr(), ws.numel(), None)
        torch.cuda.synchronize()
        outs.append(out.float().cpu().numpy())
    assert om.normwise_rel(outs[1], outs[0]) <= 2 ** -8


@pytest.mark.parametrize("hidden,heads,q_lora,gate", [(1024, 16, 512, False), (768, 4, 1536, True),
                                                      (9216, 80, 512, True)])
def test_mla_fused_decode_step_other_shapes(hidden, heads, q_lora, gate):
    """Other head counts, q_lora ranks and no output gate: the fused step against the
    fp64 restatement on the latents it stored, nine tokens from an empty cache.  Hidden 9216
    with 80 heads sends the x rows (q_a, kv_a, g_proj over 9216 values) and the o_proj rows
    (over 80 x 128 = 10240 values) through the dense row kernel's widest per-block form
    (rows of 8193..12288 values, two rows per wave)."""
    from k3hip.mla import MLAAttention
    cfg = Cfg(hidden_size=hidden, num_attention_heads=heads, q_lora_rank=q_lora, mla_use_output_gate=gate)
    rng = np.random.default_rng(hidden + heads)
    w32 = {k: bf(v) for k, v in omla.random_mla_weights(rng, cfg).items()}
    wdev = {k: torch.from_numpy(v).to(DEV).to(torch.bfloat16) for k, v in w32.items()}
    attn = MLAAttention(cfg, wdev)
    assert attn.fused_step
    x = bf((rng.standard_normal((1, 9, hidden)) * 0.5).astype(np.float32))
    xd = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    cache = None
    w = {k: v.astype(np.float64) for k, v in w32.items()}
    kb = w["kv_b_proj.weight"].reshape(heads, 256, 512)
    rms = lambda a, g: g * a / np.sqrt((a * a).mean(-1, keepdims=True) + cfg.rms_norm_eps)  # noqa: E731
    worst = 0.0
    for t in range(9):
        o, cache = attn(xd[:, t:t + 1], cache=cache)
        lat = cache.latent[0, :t + 1].float().cpu().numpy().astype(np.float64)
        rot = cache.rot[0, :t + 1].float().cpu().numpy().astype(np.float64)
        q = (rms(x[0, t].astype(np.float64) @ w["q_a_proj.weight"].T, w["q_a_layernorm.weight"])
             @ w["q_b_proj.weight"].T).reshape(heads, 192)
        oo = omla.mla_decode_absorbed(q[:, :128], q[:, 128:], kb[:, :128], kb[:, 128:], lat, rot,
                                      192 ** -0.5)[0].reshape(-1)
        if gate:
            oo = oo / (1.0 + np.exp(-(x[0, t].astype(np.float64) @ w["g_proj.weight"].T)))
        worst = max(worst, om.normwise_rel(o.float().cpu().numpy().reshape(-1), oo @ w["o_proj.weight"].T))
    print(f"hidden={hidden} heads={heads} q_lora={q_lora} gate={gate}: {worst:.2e}")
    assert worst <= 1e-4
