"""The multi-token (prefill) form of MLAAttention on the host: its query chunks, taken so
that no chunk's fp32 scores exceed MLAAttention.DENSE_SCORE_BYTES, give the causal absorbed
attention of the whole block (attention_mla.py:193-212 for each query row, with the causal
mask of the prompt) within fp32 rounding of an fp64 restatement, whatever the chunk size."""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from k3hip.mla import MLAAttention


def _stub(nope, wk, wv, budget):
    return SimpleNamespace(cfg=SimpleNamespace(qk_nope_head_dim=nope), _wk32=wk, _wv32=wv,
                           DENSE_SCORE_BYTES=budget)


def _fp64(q, lat, rot, wk, wv, scale, nope):
    """Causal absorbed attention in fp64: row t of the Tq queries sees cache rows
    0 .. Tk - Tq + t."""
    q, lat, rot, wk, wv = (a.double().numpy() for a in (q, lat, rot, wk, wv))
    B, H, Tq, _ = q.shape
    Tk = lat.shape[1]
    out = np.zeros((B, H, Tq, wv.shape[1]))
    for b in range(B):
        for h in range(H):
            for t in range(Tq):
                n = Tk - Tq + t + 1
                s = (q[b, h, t, :nope] @ wk[h]) @ lat[b, :n].T + q[b, h, t, nope:] @ rot[b, :n].T
                s = s * scale
                p = np.exp(s - s.max())
                p /= p.sum()
                out[b, h, t] = wv[h] @ (p @ lat[b, :n])
    return out


@pytest.mark.parametrize("budget", [1 << 40, 3 * 4 * 40 * 4, 4 * 4 * 40])
def test_dense_query_chunks_match_fp64(budget):
    g = torch.Generator().manual_seed(7)
    B, H, Tq, Tk, nope, rope, r, v = 1, 3, 9, 40, 16, 8, 32, 12
    q = torch.randn(B, H, Tq, nope + rope, generator=g)
    lat = torch.randn(B, Tk, r, generator=g)
    rot = torch.randn(B, Tk, rope, generator=g)
    wk = torch.randn(H, nope, r, generator=g) * 0.2
    wv = torch.randn(H, v, r, generator=g) * 0.2
    scale = (nope + rope) ** -0.5
    got = MLAAttention._dense(_stub(nope, wk, wv, budget), q, lat, rot, scale)
    want = _fp64(q, lat, rot, wk, wv, scale, nope)
    assert got.shape == (B, H, Tq, v)
    err = np.abs(got.double().numpy() - want).max() / np.abs(want).max()
    assert err < 1e-5, err


def test_dense_chunk_size_from_budget():
    """A budget of three query rows' scores runs the prompt in chunks of three (the last one
    short), and the rows equal the one-chunk result."""
    g = torch.Generator().manual_seed(8)
    B, H, Tq, Tk, nope, rope, r, v = 1, 2, 8, 20, 8, 4, 16, 6
    q = torch.randn(B, H, Tq, nope + rope, generator=g)
    lat, rot = torch.randn(B, Tk, r, generator=g), torch.randn(B, Tk, rope, generator=g)
    wk, wv = torch.randn(H, nope, r, generator=g), torch.randn(H, v, r, generator=g)
    one = MLAAttention._dense(_stub(nope, wk, wv, 1 << 40), q, lat, rot, 0.3)
    three = MLAAttention._dense(_stub(nope, wk, wv, B * H * Tk * 4 * 3), q, lat, rot, 0.3)
    # the same products in other matmul shapes: equal to fp32 rounding
    assert (one - three).abs().max() <= 1e-6 * one.abs().max()
