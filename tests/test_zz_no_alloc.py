"""The allocation-free expert FFN (k3_expert_ffn_noalloc) against k3_expert_ffn, through
the C-ABI: same kernels, so the outputs must be bit-identical.  Two calls in a row, the
second with a smaller expert (the scratch keeps the first call's act values, which the
second call must overwrite or ignore), then a size past the scratch, which is refused on the
host before anything is launched."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _expert(seed, H, I):
    rng = np.random.default_rng(seed)
    mats = [om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, I, H), om.random_mxfp4(rng, H, I)]
    x = om.bf16_round(rng.standard_normal((1, H)).astype(np.float32))
    dev = [tuple(torch.from_numpy(a).to(DEV) for a in m) for m in mats]
    return torch.from_numpy(x).to(DEV).to(torch.bfloat16), dev


def _call(name, x, mats, H, I, out, ws=None, act=0, beta=1.0, lbeta=0.0):
    from k3hip import _lib
    from k3hip import _torch as T
    (gp, gs), (up, us), (dp, ds) = mats
    args = [T.ptr(x), _lib.K3_BF16, T.ptr(gp), T.ptr(gs), T.ptr(up), T.ptr(us), T.ptr(dp), T.ptr(ds), T.ptr(out),
            _lib.K3_F32, H, I, act, float(beta), float(lbeta)]
    if ws is not None:
        args += [T.ptr(ws), ws.numel()]
    _lib.call(name, *args, T.stream(x))


def _reference(x, mats, H, I, act=0, beta=1.0, lbeta=0.0):
    from k3hip import _lib
    ws = torch.zeros(int(_lib.lib().k3_expert_ffn_workspace_size(I)), dtype=torch.uint8, device=DEV)
    out = torch.empty(1, H, device=DEV)
    _call("k3_expert_ffn", x, mats, H, I, out, ws, act, beta, lbeta)
    return out


def test_noalloc_matches_workspace_entry_point_twice_then_smaller():
    for seed, H, I, act in ((1, 7168, 2048, 0), (2, 1024, 256, 1)):   # second call: a smaller expert
        x, mats = _expert(seed, H, I)
        out = torch.full((1, H), float("nan"), device=DEV)
        _call("k3_expert_ffn_noalloc", x, mats, H, I, out, act=act, beta=2.0, lbeta=3.0)
        want = _reference(x, mats, H, I, act, 2.0, 3.0)
        torch.cuda.synchronize()
        print(f"H={H} I={I}: max |diff| {(out - want).abs().max().item():.3e}")
        assert torch.equal(out, want)


def test_noalloc_rejects_sizes_past_its_scratch():
    from k3hip import _lib
    H, I = 256, 16384 + 128
    x = torch.zeros(1, H, dtype=torch.bfloat16, device=DEV)
    mats = [(torch.zeros(I, H // 2, dtype=torch.uint8, device=DEV), torch.zeros(I, H // 32, dtype=torch.uint8,
                                                                                   device=DEV)),
            (torch.zeros(I, H // 2, dtype=torch.uint8, device=DEV), torch.zeros(I, H // 32, dtype=torch.uint8,
                                                                                   device=DEV)),
            (torch.zeros(H, I // 2, dtype=torch.uint8, device=DEV), torch.zeros(H, I // 32, dtype=torch.uint8,
                                                                                   device=DEV))]
    out = torch.empty(1, H, device=DEV)
    with pytest.raises(ValueError, match="scratch"):
        _call("k3_expert_ffn_noalloc", x, mats, H, I, out)
    assert b"16384" in _lib.lib().k3_last_error()
