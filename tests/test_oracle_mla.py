"""Pin the latent-MLA oracle (CPU only).

Every check compares the oracle with something that does not share its formula: a
pure-Python loop written from the attention definition, the expanded (per-head K/V) form
the absorbed one must equal (the reference's gate N3, tests/test_mla_cache.py:258-274),
closed-form special cases, and the layer oracle's last row against the decode core.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import pytest

from oracle import mla as omla


def brute_force(q_nope, q_rot, w_uk, w_uv, lat, rot, scale):
    """Definition-level loops: k_t^h = [W_UK^h lat_t ; rot_t], v_t^h = W_UV^h lat_t."""
    H, nope = len(q_nope), len(q_nope[0])
    T, r = len(lat), len(lat[0])
    out = []
    for h in range(H):
        scores = []
        vals = []
        for t in range(T):
            key = [sum(w_uk[h][n][j] * lat[t][j] for j in range(r)) for n in range(nope)]
            s = sum(q_nope[h][n] * key[n] for n in range(nope))
            s += sum(q_rot[h][j] * rot[t][j] for j in range(len(rot[t])))
            scores.append(s * scale)
            vals.append([sum(w_uv[h][v][j] * lat[t][j] for j in range(r)) for v in range(len(w_uv[h]))])
        m = max(scores)
        e = [math.exp(s - m) for s in scores]
        z = sum(e)
        out.append([sum(e[t] * vals[t][v] for t in range(T)) / z for v in range(len(vals[0]))])
    return np.array(out)


def rand_core(rng, H, nope, rope, r, v, T):
    return (rng.standard_normal((H, nope)), rng.standard_normal((H, rope)),
            rng.standard_normal((H, nope, r)) * 0.3, rng.standard_normal((H, v, r)) * 0.3,
            rng.standard_normal((T, r)), rng.standard_normal((T, rope)))


def test_absorbed_matches_brute_force_loops():
    rng = np.random.default_rng(0)
    args = rand_core(rng, H=3, nope=4, rope=2, r=5, v=3, T=6)
    got = omla.mla_decode_absorbed(*args, scale=0.37)[0]
    want = brute_force(*(a.tolist() for a in args), 0.37)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("T", [1, 7, 300])
def test_absorbed_equals_expanded(T):
    """Gate N3 (tests/test_mla_cache.py:258-274) at the real head dims."""
    rng = np.random.default_rng(T)
    args = rand_core(rng, H=4, nope=128, rope=64, r=512, v=128, T=T)
    a = omla.mla_decode_absorbed(*args, scale=192 ** -0.5)[0]
    e = omla.mla_decode_expanded(*args, scale=192 ** -0.5)
    np.testing.assert_allclose(a, e, rtol=1e-10, atol=1e-10)


def test_single_token_returns_projected_latent():
    rng = np.random.default_rng(1)
    q_nope, q_rot, w_uk, w_uv, lat, rot = rand_core(rng, 4, 8, 4, 16, 8, 1)
    out = omla.mla_decode_absorbed(q_nope, q_rot, w_uk, w_uv, lat, rot, 0.2)[0]
    want = np.einsum("hvr,r->hv", w_uv, lat[0])
    np.testing.assert_allclose(out, want, rtol=1e-13)


def test_shared_rope_key_is_a_per_head_constant():
    """All tokens share one rot vector: q_rot . rot is constant per head, so the output
    must not depend on q_rot (softmax is shift-invariant)."""
    rng = np.random.default_rng(2)
    q_nope, q_rot, w_uk, w_uv, lat, rot = rand_core(rng, 3, 8, 4, 16, 8, 20)
    rot[:] = rot[0]
    a = omla.mla_decode_absorbed(q_nope, q_rot, w_uk, w_uv, lat, rot, 0.3)[0]
    b = omla.mla_decode_absorbed(q_nope, 5.0 * rng.standard_normal(q_rot.shape), w_uk, w_uv, lat, rot, 0.3)[0]
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12)


def test_identical_tokens_equal_one_token():
    rng = np.random.default_rng(3)
    q_nope, q_rot, w_uk, w_uv, lat, rot = rand_core(rng, 2, 8, 4, 16, 8, 1)
    one = omla.mla_decode_absorbed(q_nope, q_rot, w_uk, w_uv, lat, rot, 0.3)[0]
    many = omla.mla_decode_absorbed(q_nope, q_rot, w_uk, w_uv, np.repeat(lat, 9, 0), np.repeat(rot, 9, 0), 0.3)[0]
    np.testing.assert_allclose(one, many, rtol=1e-13)


@pytest.mark.parametrize("splits", [1, 2, 5, 64])
def test_split_merge_equals_one_shot_softmax(splits):
    rng = np.random.default_rng(4)
    s = rng.standard_normal(200) * 3
    v = rng.standard_normal((200, 6))
    p = np.exp(s - s.max())
    np.testing.assert_allclose(omla.split_merge_softmax(s, v, splits), p @ v / p.sum(), rtol=1e-12)


@dataclass
class Cfg:
    hidden_size: int = 256
    num_attention_heads: int = 4
    q_lora_rank: int = 96
    kv_lora_rank: int = 512
    qk_nope_head_dim: int = 128
    qk_rope_head_dim: int = 64
    v_head_dim: int = 128
    rms_norm_eps: float = 1e-5
    mla_use_output_gate: bool = True

    @property
    def q_head_dim(self):
        return self.qk_nope_head_dim + self.qk_rope_head_dim


def test_layer_last_row_equals_decode_core():
    """The layer oracle's last query sees every position (causal_mask places queries at
    the end, attention_mla.py:200-207), so its row must equal projections + the absorbed
    decode core on the full latent cache: pins the mask and the kv_b split together."""
    cfg = Cfg()
    rng = np.random.default_rng(5)
    w = {k: v.astype(np.float64) for k, v in omla.random_mla_weights(rng, cfg).items()}
    x = rng.standard_normal((1, 9, cfg.hidden_size))
    full = omla.mla_layer_expanded(cfg, w, x)[0, -1]

    nh, nope, klr, vhd = cfg.num_attention_heads, cfg.qk_nope_head_dim, cfg.kv_lora_rank, cfg.v_head_dim
    rms = lambda a, g: g * a / np.sqrt((a * a).mean(-1, keepdims=True) + cfg.rms_norm_eps)  # noqa: E731
    q = (rms(x[0, -1] @ w["q_a_proj.weight"].T, w["q_a_layernorm.weight"]) @ w["q_b_proj.weight"].T)
    q = q.reshape(nh, cfg.q_head_dim)
    ckv = x[0] @ w["kv_a_proj_with_mqa.weight"].T
    lat = rms(ckv[:, :klr], w["kv_a_layernorm.weight"])
    kb = w["kv_b_proj.weight"].reshape(nh, nope + vhd, klr)
    o = omla.mla_decode_absorbed(q[:, :nope], q[:, nope:], kb[:, :nope], kb[:, nope:], lat, ckv[:, klr:],
                                 cfg.q_head_dim ** -0.5)[0].reshape(-1)
    o = o / (1.0 + np.exp(-(x[0, -1] @ w["g_proj.weight"].T)))
    np.testing.assert_allclose(full, o @ w["o_proj.weight"].T, rtol=1e-10, atol=1e-12)


def test_planted_transpose_is_caught():
    """A plausible slip (W_UV applied transposed per head) must fail the brute-force check."""
    rng = np.random.default_rng(6)
    q_nope, q_rot, w_uk, w_uv, lat, rot = rand_core(rng, 2, 4, 2, 4, 4, 5)
    good = brute_force(*(a.tolist() for a in (q_nope, q_rot, w_uk, w_uv, lat, rot)), 0.5)
    bad = omla.mla_decode_absorbed(q_nope, q_rot, w_uk, w_uv.transpose(0, 2, 1), lat, rot, 0.5)[0]
    assert not np.allclose(bad, good, rtol=1e-6)
