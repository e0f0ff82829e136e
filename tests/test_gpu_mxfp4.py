"""GPU parity: MXFP4 decode (bit-exact) and the fused matvec (vs the fp64 oracle and the
reference's unfused dequant-then-matmul definition).  Calls go through the C-ABI."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _bf16_tensor(a32: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a32, dtype=np.float32)).to(torch.bfloat16).to(DEV)


# ------------------------------------------------------------------------- decode

def test_decode_truth_table_bit_exact():
    from k3hip.mxfp4 import decode_mxfp4
    codes = np.arange(16, dtype=np.uint8)
    packed = np.zeros((256, 16), dtype=np.uint8)
    packed[:, :8] = (codes[0::2] | (codes[1::2] << 4))[None, :]
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    want = om.decode_mxfp4(packed, scales)
    for dt in (torch.float32, torch.bfloat16):
        got = decode_mxfp4(_t(packed), _t(scales), out_dtype=dt).float().cpu().numpy()
        w = want if dt == torch.float32 else om.bf16_round(want)
        nan = np.isnan(w)
        assert np.array_equal(np.isnan(got), nan), dt
        assert np.array_equal(got.view(np.uint32)[~nan], w.view(np.uint32)[~nan]), dt


@pytest.mark.parametrize("n,k", [(1, 32), (3, 96), (64, 512), (2048, 7168)])
def test_decode_random_bit_exact(n, k):
    from k3hip.mxfp4 import decode_mxfp4, decode_mxfp4_mlx
    rng = np.random.default_rng(n * 7 + k)
    packed = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = rng.integers(1, 255, size=(n, k // 32), dtype=np.uint8)
    want = om.decode_mxfp4(packed, scales)
    got = decode_mxfp4(_t(packed), _t(scales)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = decode_mxfp4_mlx(_t(packed), _t(scales), out_dtype=torch.bfloat16)
    assert np.array_equal(got16.float().cpu().numpy(), want)   # lossless in bf16


def test_scale_guard():
    from k3hip.mxfp4 import assert_scales_representable, decode_scale
    ok = torch.tensor([[2, 120, 252]], dtype=torch.uint8, device=DEV)
    assert_scales_representable(ok)
    for bad in (0, 1, 253, 255):
        with pytest.raises(ValueError, match="scale range"):
            assert_scales_representable(torch.tensor([[120, bad]], dtype=torch.uint8, device=DEV))
    b = np.arange(256, dtype=np.uint8)
    got = decode_scale(_t(b)).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), om.e8m0_to_f32(b).view(np.uint32))


# ------------------------------------------------------------------------- matvec

def _case(seed, n, k, m, lo=118, hi=130):
    rng = np.random.default_rng(seed)
    packed, scales = om.random_mxfp4(rng, n, k, lo, hi)
    x = rng.standard_normal((m, k)).astype(np.float32)
    return packed, scales, x


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 9])
def test_matvec_reference_synthetic_gate(m, xdt):
    """tests/test_mxfp4_kernel.py:42-54: N=128, K=256, packed uniform, scales [100,140),
    x ~ N(0,1); normwise rel < 1e-6 vs the fp64 oracle."""
    from k3hip.mxfp4_matvec import mxfp4_matvec_fused
    rng = np.random.default_rng(0)
    packed = rng.integers(0, 256, size=(128, 128), dtype=np.uint8)
    scales = rng.integers(100, 140, size=(128, 8), dtype=np.uint8)
    x32 = rng.standard_normal((m, 256)).astype(np.float32)
    if xdt == torch.bfloat16:
        x32 = om.bf16_round(x32)
    x = torch.from_numpy(x32).to(DEV).to(xdt)
    got = mxfp4_matvec_fused(x, _t(packed), _t(scales)).cpu().numpy()
    want = om.matvec_f64(x32, packed, scales)
    assert om.normwise_rel(got, want) < 1e-6


SHAPES = [(1, 32), (7, 64), (129, 96), (300, 480), (2048, 7168), (7168, 2048), (384, 7168),
          (3072, 3584), (3584, 3072), (1000, 8192), (64, 16384)]


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_matvec_shapes_vs_oracle(n, k, xdt):
    from k3hip.mxfp4_matvec import mxfp4_matvec_fused
    packed, scales, x32 = _case(n + k, n, k, 1)
    if xdt == torch.bfloat16:
        x32 = om.bf16_round(x32)
    x = torch.from_numpy(x32).to(DEV).to(xdt)
    got = mxfp4_matvec_fused(x, _t(packed), _t(scales)).cpu().numpy()
    want = om.matvec_f64(x32, packed, scales)
    assert om.normwise_rel(got, want) < 2e-6
    unfused = om.matvec_unfused_f64(x32, packed, scales)
    if xdt == torch.bfloat16:
        # the gate on the configured (bf16) activations: within 1e-3 of the reference's
        # own dequant-then-matmul (air_llm/models/kimi_k3/mxfp4.py:84-92)
        assert om.normwise_rel(got, unfused) <= 1e-3
    else:
        # fp32 activations: that definition rounds x to bf16 first, so the fused result
        # must be at least as accurate as it (tests/test_mxfp4_kernel.py:70-84)
        assert om.normwise_rel(got, want) <= om.normwise_rel(unfused, want)


# (N, K) pairs that select every default launch shape (rows per wave, 32-element groups per
# lane per sweep): gpl 1 / 2 / 4 by K, rows per wave by N; K = 16384 sweeps each row twice.
LAUNCH_SHAPES = [(500, 2048), (1040, 2048), (4100, 1024), (8200, 512), (500, 3072), (2100, 3072), (4100, 3072),
                 (500, 7168), (8200, 7168), (300, 16384)]


@pytest.mark.parametrize("N,K", LAUNCH_SHAPES)
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
def test_matvec_every_launch_shape(N, K, xdt):
    """Every (rows per wave, groups per lane) the default configuration picks, with N not
    a multiple of the rows per block (tail rows read zeros and are not stored)."""
    from k3hip.mxfp4_matvec import mxfp4_matvec_fused
    packed, scales, x32 = _case(N + K, N, K, 1)
    if xdt == torch.bfloat16:
        x32 = om.bf16_round(x32)
    x = torch.from_numpy(x32).to(DEV).to(xdt)
    got = mxfp4_matvec_fused(x, _t(packed), _t(scales)).cpu().numpy()
    assert om.normwise_rel(got, om.matvec_f64(x32, packed, scales)) < 2e-6


@pytest.mark.parametrize("n,k", [(2048, 7168), (7168, 2048)])
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("band", ["low", "high", "mixed"])
def test_matvec_scale_bytes_at_the_legal_edges(n, k, xdt, band):
    """Scale bytes at both ends of the accepted range 2..252 (mxfp4.py:58-65): 2..20 (block
    scales down to 2^-125, products down to 2^-126, the smallest normal fp32 / bf16 value),
    240..252 (up to 2^125, products up to 1.5 x 2^127) with x scaled by 2^-24 so the sums
    stay finite, and rows mixing both ends group by group."""
    from k3hip.mxfp4_matvec import mxfp4_matvec_fused
    rng = np.random.default_rng(n + 3 * k + {"low": 0, "high": 1, "mixed": 2}[band])
    packed = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    lo_s = rng.integers(2, 21, size=(n, k // 32), dtype=np.uint8)
    hi_s = rng.integers(240, 253, size=(n, k // 32), dtype=np.uint8)
    scales = {"low": lo_s, "high": hi_s, "mixed": np.where(rng.random((n, k // 32)) < 0.5, lo_s, hi_s)}[band]
    x32 = rng.standard_normal((1, k)).astype(np.float32) * np.float32(2.0 ** (-24 if band != "low" else 0))
    if xdt == torch.bfloat16:
        x32 = om.bf16_round(x32)
    x = torch.from_numpy(x32).to(DEV).to(xdt)
    got = mxfp4_matvec_fused(x, _t(packed), _t(scales)).cpu().numpy()
    want = om.matvec_f64(x32, packed, scales)
    assert np.isfinite(got).all() and np.isfinite(want).all()
    assert om.normwise_rel(got, want) < 2e-6


def test_matvec_bf16_output_is_rne_of_fp32():
    from k3hip.mxfp4_matvec import mxfp4_matvec_fused
    packed, scales, x32 = _case(1001, 2048, 7168, 1)
    x = _bf16_tensor(x32)
    P, S = _t(packed), _t(scales)
    f = mxfp4_matvec_fused(x, P, S).cpu().numpy()
    b = mxfp4_matvec_fused(x, P, S, out_dtype=torch.bfloat16).float().cpu().numpy()
    assert np.array_equal(b.view(np.uint32), om.bf16_round(f).view(np.uint32))


def test_matvec_deterministic():
    from k3hip.mxfp4_matvec import mxfp4_matvec_fused
    packed, scales, x32 = _case(77, 2048, 7168, 1)
    x, P, S = _bf16_tensor(x32), _t(packed), _t(scales)
    a = mxfp4_matvec_fused(x, P, S)
    for _ in range(3):
        assert torch.equal(a, mxfp4_matvec_fused(x, P, S))


def test_matvec_zero_rows_and_empty():
    from k3hip.mxfp4_matvec import expert_projection, mxfp4_matvec_fused
    packed, scales, x32 = _case(3, 16, 64, 1)
    x = torch.from_numpy(x32).to(DEV)
    assert mxfp4_matvec_fused(x[:0], _t(packed), _t(scales)).shape == (0, 16)
    y1 = expert_projection(x[0], _t(packed), _t(scales))
    assert y1.shape == (16,)
    assert om.normwise_rel(y1.cpu().numpy(), om.matvec_f64(x32[0], packed, scales)) < 2e-6


def test_matvec_errors_match_reference():
    from k3hip.mxfp4_matvec import mxfp4_matvec_fused
    packed, scales, x32 = _case(4, 16, 64, 1)
    with pytest.raises(ValueError, match="K mismatch"):
        mxfp4_matvec_fused(torch.zeros(1, 96, device=DEV), _t(packed), _t(scales))


def test_unfused_path_matches_definition():
    from k3hip.mxfp4 import mxfp4_matvec
    packed, scales, x32 = _case(5, 256, 1024, 2)
    got = mxfp4_matvec(torch.from_numpy(x32).to(DEV), _t(packed), _t(scales)).cpu().numpy()
    # a bf16 x bf16 matmul returns bf16 (as MLX's does in mxfp4.py:92), so the unfused
    # result carries one bf16 output rounding on top of the exact contraction
    want = om.matvec_unfused_f64(x32, packed, scales)
    assert np.all(np.abs(got - want) <= np.abs(want) * 2.0 ** -8 + 1e-6)
