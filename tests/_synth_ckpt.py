"""Synthetic K3 MoE checkpoint shards for the ingestion tests: the reference's tensor
names (loader.py:30-33, 238-239), MXFP4 experts from the oracle's encoder (the fixture
generator of tools/make_synthetic_k3.py:87-110, restated in oracle/mxfp4.py), dense
weights as bf16 bit patterns."""
from __future__ import annotations

import numpy as np

from oracle import mxfp4 as om


def _bf16(rng, shape, std):
    return om.bf16_bits(rng.standard_normal(shape).astype(np.float32) * std)


def make_k3_checkpoint(root, seed, layer, H, L, I, E, Is, gap_expert=None, bad_scale=None):
    """Write two shards under root; expert e's projections go to shard e * 2 // E.  Every
    (packed, scale) pair is adjacent except expert ``gap_expert``'s w3, whose scale sits
    after its w2 pair.  ``bad_scale`` = (expert, which) sets one scale byte to 255.
    Returns the arrays the oracle needs (dense weights as float32 values)."""
    from k3hip.checkpoint import expert_name, moe_prefix, write_safetensors
    rng = np.random.default_rng(seed)
    dense = {"gate.weight": (_bf16(rng, (E, H), 0.02), "BF16"),
             "gate.e_score_correction_bias": ((rng.standard_normal(E) * 0.05).astype(np.float32), "F32"),
             "routed_expert_down_proj.weight": (_bf16(rng, (L, H), 0.02), "BF16"),
             "routed_expert_up_proj.weight": (_bf16(rng, (H, L), 0.02), "BF16"),
             "routed_expert_norm.weight": ((1.0 + 0.1 * rng.standard_normal(L)).astype(np.float32), "F32"),
             "shared_experts.gate_proj.weight": (_bf16(rng, (Is, H), 0.02), "BF16"),
             "shared_experts.up_proj.weight": (_bf16(rng, (Is, H), 0.02), "BF16"),
             "shared_experts.down_proj.weight": (_bf16(rng, (H, Is), 0.02), "BF16")}
    shapes = {"w1": (I, L), "w3": (I, L), "w2": (L, I)}
    experts = {}
    shards = [{moe_prefix(layer) + k: v for k, v in dense.items()}, {}]
    for e in range(E):
        proj = {}
        for w in ("w1", "w3", "w2"):
            p, s = om.encode_mxfp4(rng.standard_normal(shapes[w]).astype(np.float32) * 0.05)
            if bad_scale == (e, w):
                s = s.copy()
                s[0, 0] = 255
            proj[w] = (p, s)
        experts[e] = (proj["w1"], proj["w3"], proj["w2"])
        out = shards[e * 2 // E]
        order = ["w1", "w3", "w2"]
        for w in order:
            base = expert_name(layer, e, w)
            out[base + ".weight_packed"] = (proj[w][0], "U8")
            if not (e == gap_expert and w == "w3"):
                out[base + ".weight_scale"] = (proj[w][1], "U8")
        if e == gap_expert:
            out[expert_name(layer, e, "w3") + ".weight_scale"] = (proj["w3"][1], "U8")
    for j, t in enumerate(shards):
        write_safetensors(root / f"model-{j + 1:05d}-of-00002.safetensors", t)
    f = {k: (om.bf16_from_bits(a) if dt == "BF16" else a) for k, (a, dt) in dense.items()}
    shared = (f["shared_experts.gate_proj.weight"], f["shared_experts.up_proj.weight"],
              f["shared_experts.down_proj.weight"])
    return {"dense": f, "experts": experts, "shared": shared}
