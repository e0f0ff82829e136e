"""Write the golden fixtures under tests/golden/ (run from the repository root):

    python tests/golden/make_golden.py

Each fixture is a compressed .npz of plain arrays (no pickles): seeded inputs, with bf16
values stored as uint16 bit patterns so the GPU path reads exactly the same numbers, and
the expected outputs.

* ``mxfp4_kat.npz``     the reference's two decode known-answer tests
                        (tests/test_mxfp4_mlx.py:33-61): every packed byte at scale 127,
                        every scale byte with packed 0x22.  Expected values come from the
                        closed form (exact rationals), not from the oracle.
* ``matvec_n128_k256.npz`` the reference's synthetic kernel gate
                        (tests/test_mxfp4_kernel.py:42-54): default_rng(0), N=128, K=256,
                        packed uniform 0..255, scales uniform [100, 140), x ~ N(0,1), M=4;
                        expected = fp64 product on the exactly decoded weights.
* ``expert_h256_i128.npz``  one SwiGLU expert (and one SiTU variant) at batch 1.
* ``moe_layer_h128.npz``    softmax top-2 of 6 experts + a bf16 shared expert, 3 tokens.
* ``mla_h2_t24.npz``        absorbed latent-MLA decode, 2 heads, 24 cached tokens,
                            kv_lora_rank 512, rope 64, nope 32, v 32, scale 1/sqrt(192).

Outputs other than the KATs come from the fp64 oracle in ``oracle/``; the oracle itself is
pinned by tests/test_oracle_*.py.  Re-running rewrites identical files.
"""
from __future__ import annotations

import sys
from fractions import Fraction
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from oracle import mla as omla  # noqa: E402
from oracle import moe as omoe  # noqa: E402
from oracle import mxfp4 as om  # noqa: E402

MAG = [Fraction(0), Fraction(1, 2), Fraction(1), Fraction(3, 2), Fraction(2), Fraction(3), Fraction(4), Fraction(6)]


def closed_form(code: int, sbyte: int) -> np.float32:
    """E2M1 code x 2^(sbyte-127) for bytes 1..254 (finite, normal or exact subnormal)."""
    v = MAG[code & 7] * Fraction(2) ** (sbyte - 127)
    f = np.float32(float(v))
    return np.float32(-f) if code & 8 else f


def bf16_bits(a):
    return om.bf16_bits(np.asarray(a, np.float32))


def bf16_vals(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def kat():
    packed = np.arange(256, dtype=np.uint8).reshape(1, 256)            # every packed byte
    scales = np.full((1, 16), 127, dtype=np.uint8)
    want_p = np.array([closed_form(b & 15, 127) if i == 0 else closed_form(b >> 4, 127)
                       for b in range(256) for i in (0, 1)], dtype=np.float32).reshape(1, 512)
    sbytes = np.arange(1, 255, dtype=np.uint8)                           # every finite scale byte
    packed_s = np.full((254, 16), 0x22, dtype=np.uint8)
    scales_s = sbytes.reshape(254, 1)
    want_s = np.array([closed_form(2, int(s)) for s in sbytes], dtype=np.float32)
    return dict(packed=packed, scales=scales, want_bits=want_p.view(np.uint32),
                packed_s=packed_s, scales_s=scales_s, want_s_bits=want_s.view(np.uint32))


def matvec():
    rng = np.random.default_rng(0)
    n, k = 128, 256
    packed = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = rng.integers(100, 140, size=(n, k // 32), dtype=np.uint8)
    x = rng.standard_normal((4, k)).astype(np.float32)
    return dict(packed=packed, scales=scales, x=x, want=om.matvec_f64(x, packed, scales))


def expert():
    rng = np.random.default_rng(1002)
    H, I = 256, 128
    gate, up, down = om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, H, I)
    xb = bf16_bits(rng.standard_normal((1, H)))
    x = bf16_vals(xb)
    return dict(gp=gate[0], gs=gate[1], up=up[0], us=up[1], dp=down[0], ds=down[1], x_bf16=xb,
                want_silu=omoe.expert_ffn(x, gate, up, down, "silu")[0],
                want_situ=omoe.expert_ffn(x, gate, up, down, "situ", beta=2.0, linear_beta=3.0)[0])


def layer():
    rng = np.random.default_rng(1003)
    H, I, E, k, Is, T = 128, 128, 6, 2, 128, 3
    ex = [(om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, H, I)) for _ in range(E)]
    rb = bf16_bits(rng.standard_normal((E, H)) * 0.3)
    sh = [bf16_bits(rng.standard_normal(s) * 0.05) for s in ((Is, H), (Is, H), (H, Is))]
    xb = bf16_bits(rng.standard_normal((T, H)))
    x = bf16_vals(xb).astype(np.float64)
    idx, w, probs, _ = omoe.route_softmax(x, bf16_vals(rb), k)
    y = omoe.moe_layer(x, idx, w, ex, shared=tuple(bf16_vals(s) for s in sh))
    d = dict(x_bf16=xb, router_bf16=rb, sh_gate_bf16=sh[0], sh_up_bf16=sh[1], sh_down_bf16=sh[2],
             want=y, want_idx=idx.astype(np.int64), want_w=w, want_probs=probs)
    for e, (g, u, dn) in enumerate(ex):
        d.update({f"e{e}_gp": g[0], f"e{e}_gs": g[1], f"e{e}_up": u[0], f"e{e}_us": u[1],
                  f"e{e}_dp": dn[0], f"e{e}_ds": dn[1]})
    return d


def mla():
    rng = np.random.default_rng(1005)
    H, T, nope, v = 2, 24, 32, 32
    arrs = dict(q_nope=rng.standard_normal((H, nope)), q_rot=rng.standard_normal((H, 64)),
                w_uk=rng.standard_normal((H, nope, 512)) * 0.02, w_uv=rng.standard_normal((H, v, 512)) * 0.02,
                lat=rng.standard_normal((T, 512)), rot=rng.standard_normal((T, 64)))
    bits = {f"{k}_bf16": bf16_bits(a) for k, a in arrs.items()}
    vals = [bf16_vals(bits[f"{k}_bf16"]) for k in arrs]
    bits["want"] = omla.mla_decode_absorbed(*vals, 192 ** -0.5)[0]
    return bits


FIXTURES = {"mxfp4_kat": kat, "matvec_n128_k256": matvec, "expert_h256_i128": expert,
            "moe_layer_h128": layer, "mla_h2_t24": mla}


def main():
    for name, fn in FIXTURES.items():
        np.savez_compressed(HERE / f"{name}.npz", **fn())
        print(f"wrote {name}.npz ({(HERE / f'{name}.npz').stat().st_size} bytes)")


if __name__ == "__main__":
    main()
