"""The miniature Kimi-K3 used by the GPU integration gate, checked on the CPU: the
checkpoint it writes reads back bit-exactly through the checkpoint reader under the
reference's tensor names, and the fp64 oracle stack generates a non-degenerate greedy
stream whose top-2 logit gaps leave room for fp32/bf16 paths to agree."""
from __future__ import annotations

import numpy as np

from _mini_k3 import NTOK, PROMPT, MiniCfg, OracleModel, build_checkpoint, layer_prefix


def test_checkpoint_round_trip_and_oracle_stream(tmp_path):
    from k3hip.checkpoint import TensorSource, expert_name

    tensors = build_checkpoint(tmp_path)
    src = TensorSource(ckpt=tmp_path)
    cfg = MiniCfg()
    for name in (layer_prefix(0) + "self_attn.q_proj.weight", layer_prefix(0) + "self_attn.A_log",
                 layer_prefix(2) + "self_attn.kv_b_proj.weight",
                 layer_prefix(1) + "block_sparse_moe.gate.e_score_correction_bias",
                 "language_model.lm_head.weight"):
        arr, _ = tensors[name]
        assert np.array_equal(src.host(name).reshape(arr.shape), arr), name
    for L in (1, 2):
        for w in ("w1", "w3", "w2"):
            packed, scales = src.expert_host(L, cfg.num_experts - 1, w)
            stem = expert_name(L, cfg.num_experts - 1, w)
            assert np.array_equal(packed, tensors[stem + ".weight_packed"][0])
            assert np.array_equal(scales, tensors[stem + ".weight_scale"][0])
            assert 2 <= scales.min() and scales.max() <= 252

    o = OracleModel(tensors)
    toks, ids, gaps = [], list(PROMPT), []
    for _ in range(NTOK):
        lg = o.logits(ids)
        assert np.all(np.isfinite(lg))
        top = np.sort(lg)[-2:]
        gaps.append((top[1] - top[0]) / np.abs(lg).max())
        toks.append(int(np.argmax(lg)))
        ids.append(toks[-1])
    assert len(set(toks)) > 1, toks
    assert min(gaps) > 1e-4, gaps
