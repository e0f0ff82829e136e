"""GPU parity of the KDA recurrent step (k3_kda_recurrent_decode) against the fp64 oracle
(oracle/kda.py, restating attention_kda.py:65-90).  fp32 state and arithmetic; the bar is
normwise max-relative 1e-5 per step for output and state, over multi-step sequences (the
state carries every step's rounding forward)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kda as okda
from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-5


def _inputs(rng, B, Tn, H, HV, K=128, V=128):
    q = okda.l2norm(rng.standard_normal((B, Tn, H, K))).astype(np.float32)
    k = okda.l2norm(rng.standard_normal((B, Tn, H, K))).astype(np.float32)
    v = rng.standard_normal((B, Tn, HV, V)).astype(np.float32)
    g = (-5.0 / (1.0 + np.exp(-rng.standard_normal((B, Tn, HV, K))))).astype(np.float32)
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((B, Tn, HV))))).astype(np.float32)
    S0 = (rng.standard_normal((B, HV, K, V)) * 0.5).astype(np.float32)
    return q, k, v, g, beta, S0


def _dev(*a, dtype=torch.float32):
    return [torch.from_numpy(np.ascontiguousarray(x)).to(DEV).to(dtype) for x in a]


@pytest.mark.parametrize("B,Tn,H,HV,V", [(1, 1, 96, 96, 128), (1, 5, 4, 4, 128), (2, 3, 3, 6, 64), (1, 2, 2, 2, 256)])
def test_kda_matches_oracle(B, Tn, H, HV, V):
    from k3hip.kda import kda_recurrent
    rng = np.random.default_rng(B * 100 + Tn * 10 + HV)
    q, k, v, g, beta, S0 = _inputs(rng, B, Tn, H, HV, V=V)
    o, S = kda_recurrent(*_dev(q, k, v, g, beta), state=_dev(S0)[0])
    want_o, want_S = okda.kda_recurrent(q, k, v, g, beta, None, S0)
    ro = om.normwise_rel(o.cpu().numpy(), want_o)
    rs = om.normwise_rel(S.cpu().numpy(), want_S)
    print(f"B={B} T={Tn} H={H} HV={HV} V={V}: out {ro:.2e} state {rs:.2e}")
    assert ro <= TOL and rs <= TOL


def test_kda_bf16_inputs_zero_state_and_in_place():
    """bf16 q/k/v/g/beta (read as their bf16 values); no initial state; the fp32 state
    passed back in is updated in place; the delta rule at beta = 1 writes v at the key."""
    from k3hip.kda import kda_recurrent
    rng = np.random.default_rng(7)
    q, k, v, g, beta, _ = _inputs(rng, 1, 1, 8, 8)
    qb, kb, vb, gb, bb = (om.bf16_round(a) for a in (q, k, v, g, beta))
    o, S = kda_recurrent(*_dev(qb, kb, vb, gb, bb, dtype=torch.bfloat16))
    want_o, want_S = okda.kda_recurrent(qb, kb, vb, gb, bb, None, None)
    assert om.normwise_rel(o.cpu().numpy(), want_o) <= TOL and om.normwise_rel(S.cpu().numpy(), want_S) <= TOL
    ptr = S.data_ptr()
    k1 = kb / np.linalg.norm(kb.astype(np.float64), axis=-1, keepdims=True).astype(np.float32)
    o2, S2 = kda_recurrent(*_dev(q, k1, v, g, np.ones_like(beta)), state=S)
    assert S2.data_ptr() == ptr
    ks = np.einsum("hk,hkv->hv", k1[0, 0].astype(np.float64), S2[0].double().cpu().numpy())
    assert np.abs(ks - v[0, 0]).max() <= 1e-4 * np.abs(v).max()


def test_kda_is_deterministic_and_validates():
    from k3hip.kda import kda_recurrent
    rng = np.random.default_rng(9)
    q, k, v, g, beta, S0 = _inputs(rng, 1, 3, 4, 4)
    a = kda_recurrent(*_dev(q, k, v, g, beta), state=_dev(S0)[0])
    b = kda_recurrent(*_dev(q, k, v, g, beta), state=_dev(S0)[0])
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    with pytest.raises(ValueError):
        kda_recurrent(*_dev(q[..., :64], k[..., :64], v, g[..., :64], beta))     # key_dim != 128
    with pytest.raises(ValueError):
        kda_recurrent(*_dev(q, k, v[..., :48], g, beta))                        # V not a multiple of 32


class KdaCfg:
    def __init__(self, hidden, heads):
        self.hidden_size, self.kda_num_heads, self.kda_head_dim, self.kda_conv_size = hidden, heads, 128, 4
        self.kda_gate_lower_bound, self.rms_norm_eps = -5.0, 1e-5


def _layer(seed, hidden, heads, scale=0.02):
    from k3hip.kda import KDAAttention
    cfg = KdaCfg(hidden, heads)
    rng = np.random.default_rng(seed)
    w = okda.random_kda_weights(rng, cfg, scale)
    for n in ("q_proj", "k_proj", "v_proj", "g_proj", "o_proj", "f_a_proj", "f_b_proj", "b_proj"):
        w[n + ".weight"] = om.bf16_round(w[n + ".weight"])                 # bf16 checkpoint weights
    wd = {n: torch.from_numpy(a).to(DEV) for n, a in w.items()}
    return cfg, w, KDAAttention(cfg, wd), rng


def test_kda_layer_steps_match_oracle_and_carry_state():
    """Five tokens from a zero state through k3_kda_step_decode against the fp64 layer; then
    the same tokens as 3 + 2 with the recurrent and convolution states carried (the
    reference's prefill == incremental gate, tests/test_k3ref_layers.py:150-168)."""
    cfg, w, attn, rng = _layer(21, 512, 4, scale=0.05)
    x = om.bf16_round(rng.standard_normal((1, 5, 512)).astype(np.float32))
    xd = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    out, S, conv = attn(xd)
    want, S_want, conv_want = okda.kda_layer(cfg, w, x)
    r_out = om.normwise_rel(out.cpu().numpy(), want)
    r_S = om.normwise_rel(S.cpu().numpy(), S_want)
    r_c = max(om.normwise_rel(a.cpu().numpy(), b) for a, b in zip(conv, conv_want))
    print(f"kda layer 5 tokens: out {r_out:.2e} state {r_S:.2e} conv {r_c:.2e}")
    assert r_out <= 2e-5 and r_S <= 2e-5 and r_c <= 1e-6
    o1, S1, c1 = attn(xd[:, :3])
    o2, S2, c2 = attn(xd[:, 3:], state=S1, conv=c1)
    assert om.normwise_rel(torch.cat([o1, o2], 1).cpu().numpy(), out.cpu().numpy()) <= 1e-6
    assert om.normwise_rel(S2.cpu().numpy(), S.cpu().numpy()) <= 1e-6


def test_kda_layer_k3_shapes_one_token():
    """K3's KDA layer shapes (hidden 7168, 96 heads of 128) for one token on a random state."""
    cfg, w, attn, rng = _layer(22, 7168, 96)
    x = om.bf16_round(rng.standard_normal((1, 1, 7168)).astype(np.float32))
    S0 = (rng.standard_normal((1, 96, 128, 128)) * 0.1).astype(np.float32)
    cv0 = tuple((rng.standard_normal((1, 3, 96 * 128)) * 0.5).astype(np.float32) for _ in range(3))
    out, S, conv = attn(torch.from_numpy(x).to(DEV).to(torch.bfloat16), state=torch.from_numpy(S0).to(DEV),
                        conv=tuple(torch.from_numpy(c).to(DEV) for c in cv0))
    want, S_want, _ = okda.kda_layer(cfg, w, x, S0, cv0)
    r_out, r_S = om.normwise_rel(out.cpu().numpy(), want), om.normwise_rel(S.cpu().numpy(), S_want)
    print(f"kda layer K3 shapes: out {r_out:.2e} state {r_S:.2e}")
    assert r_out <= 2e-5 and r_S <= 2e-5


def test_kda_layer_persistent_o_proj_odd_shapes():
    """67 heads (o_proj input 8576 wide: 17 of the lane's 24 chunk slots hold data) and hidden
    4104 (513 row groups of 8 over the persistent o_proj launch's blocks, so blocks take two
    or three groups and the last pass ends half way), one token on a random state."""
    cfg, w, attn, rng = _layer(25, 4104, 67)
    x = om.bf16_round(rng.standard_normal((1, 1, 4104)).astype(np.float32))
    S0 = (rng.standard_normal((1, 67, 128, 128)) * 0.1).astype(np.float32)
    cv0 = tuple((rng.standard_normal((1, 3, 67 * 128)) * 0.5).astype(np.float32) for _ in range(3))
    out, S, _ = attn(torch.from_numpy(x).to(DEV).to(torch.bfloat16), state=torch.from_numpy(S0).to(DEV),
                     conv=tuple(torch.from_numpy(c).to(DEV) for c in cv0))
    want, S_want, _ = okda.kda_layer(cfg, w, x, S0, cv0)
    r_out, r_S = om.normwise_rel(out.cpu().numpy(), want), om.normwise_rel(S.cpu().numpy(), S_want)
    print(f"kda layer 67 heads, hidden 4104: out {r_out:.2e} state {r_S:.2e}")
    assert r_out <= 2e-5 and r_S <= 2e-5


def test_kda_layer_batch_of_two_sequences():
    """Two sequences share the weights and keep their own recurrent and convolution states."""
    cfg, w, attn, rng = _layer(23, 256, 2, scale=0.05)
    x = om.bf16_round(rng.standard_normal((2, 3, 256)).astype(np.float32))
    out, S, conv = attn(torch.from_numpy(x).to(DEV).to(torch.bfloat16))
    want, S_want, conv_want = okda.kda_layer(cfg, w, x)
    assert om.normwise_rel(out.cpu().numpy(), want) <= 2e-5
    assert om.normwise_rel(S.cpu().numpy(), S_want) <= 2e-5
    assert max(om.normwise_rel(a.cpu().numpy(), b) for a, b in zip(conv, conv_want)) <= 1e-6
    # each sequence alone gives the same rows
    one, _, _ = attn(torch.from_numpy(x[1:]).to(DEV).to(torch.bfloat16))
    assert om.normwise_rel(one.cpu().numpy(), out[1:].cpu().numpy()) <= 1e-6


def test_kda_long_sequence_one_launch():
    """48 tokens in one launch (the state stays in registers between tokens) against the
    oracle, and equal to the same tokens split 20 + 28 across two calls."""
    from k3hip.kda import kda_recurrent
    rng = np.random.default_rng(31)
    q, k, v, g, beta, S0 = _inputs(rng, 1, 48, 16, 16)
    o, S = kda_recurrent(*_dev(q, k, v, g, beta), state=_dev(S0)[0])
    want_o, want_S = okda.kda_recurrent(q, k, v, g, beta, None, S0)
    ro, rs = om.normwise_rel(o.cpu().numpy(), want_o), om.normwise_rel(S.cpu().numpy(), want_S)
    print(f"48 tokens: out {ro:.2e} state {rs:.2e}")
    assert ro <= TOL and rs <= TOL
    sl = lambda a, i, j: a[:, i:j]  # noqa: E731
    o1, S1 = kda_recurrent(*_dev(*(sl(a, 0, 20) for a in (q, k, v, g, beta))), state=_dev(S0)[0])
    o2, S2 = kda_recurrent(*_dev(*(sl(a, 20, 48) for a in (q, k, v, g, beta))), state=S1)
    assert torch.equal(torch.cat([o1, o2], 1), o) and torch.equal(S2, S)


def test_kda_layer_other_head_count_and_fp32_input():
    """Eight heads, hidden 1024, fp32 x: three tokens against the fp64 layer."""
    cfg, w, attn, rng = _layer(24, 1024, 8, scale=0.05)
    x = rng.standard_normal((1, 3, 1024)).astype(np.float32)
    out, S, _ = attn(torch.from_numpy(x).to(DEV))
    want, S_want, _ = okda.kda_layer(cfg, w, x)
    assert om.normwise_rel(out.cpu().numpy(), want) <= 2e-5 and om.normwise_rel(S.cpu().numpy(), S_want) <= 2e-5


def test_kda_layer_prefill_path_matches_oracle_and_decode():
    """Twelve tokens take the prefill path (BLAS GEMMs + one recurrence launch); they match
    the fp64 layer, and decode tokens continue from the states it returns."""
    cfg, w, attn, rng = _layer(25, 512, 4, scale=0.05)
    x = om.bf16_round(rng.standard_normal((1, 14, 512)).astype(np.float32))
    xd = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    out, S, conv = attn(xd[:, :12])
    want, S_want, conv_want = okda.kda_layer(cfg, w, x[:, :12])
    r = om.normwise_rel(out.cpu().numpy(), want)
    print(f"kda prefill 12 tokens: {r:.2e}")
    assert r <= 2e-5 and om.normwise_rel(S.cpu().numpy(), S_want) <= 2e-5
    assert max(om.normwise_rel(a.cpu().numpy(), b) for a, b in zip(conv, conv_want)) <= 1e-6
    o2, S2, _ = attn(xd[:, 12:], state=S, conv=conv)
    want2, _, _ = okda.kda_layer(cfg, w, x[:, 12:], S_want, conv_want)
    assert om.normwise_rel(o2.cpu().numpy(), want2) <= 2e-5
