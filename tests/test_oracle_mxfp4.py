"""Pin the MXFP4 oracle (CPU only).

Each check compares the oracle with something that does not share its formula: exact
rational arithmetic, the reference's own known-answer tests restated with closed-form
expectations, an independent C restatement, or a mathematical identity.
"""
from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import mxfp4 as om
from oracle import native

MAG = [Fraction(0), Fraction(1, 2), Fraction(1), Fraction(3, 2), Fraction(2), Fraction(3),
       Fraction(4), Fraction(6)]
F32_OVERFLOW = Fraction(2) ** 128


def exact_value_bits(code: int, sbyte: int) -> int | None:
    """float32 bit pattern of E2M1 code x E8M0 byte under IEEE float32 rules; None = NaN."""
    neg = bool(code & 8)
    mag = MAG[code & 7]
    if sbyte == 255:                        # ldexp(1.0f, 128) overflows to +inf
        if mag == 0:
            return None                     # 0 * inf
        return 0xFF800000 if neg else 0x7F800000
    v = mag * Fraction(2) ** (sbyte - 127)
    if v >= F32_OVERFLOW:
        f = math.inf
    else:
        f = float(v)                        # exact: <= 3 significant bits, >= 2**-128
    f32 = np.float32(-f if neg else f)
    if mag == 0:
        f32 = np.float32(-0.0) if neg else np.float32(0.0)
    return int(np.array(f32).view(np.uint32))


def test_truth_table_all_codes_all_scales():
    codes = np.arange(16, dtype=np.uint8)
    # one row per scale byte; 16 codes in the first 16 elements of a 32-element group
    packed = np.zeros((256, 16), dtype=np.uint8)
    packed[:, :8] = (codes[0::2] | (codes[1::2] << 4))[None, :]
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    got = om.decode_mxfp4(packed, scales)[:, :16]
    bits = got.view(np.uint32)
    for s in range(256):
        for c in range(16):
            want = exact_value_bits(c, s)
            if want is None:
                assert np.isnan(got[s, c]), (s, c)
            else:
                assert int(bits[s, c]) == want, (s, c, hex(int(bits[s, c])), hex(want))


def test_kat_all_packed_bytes_scale127():
    """Restates tests/test_mxfp4_mlx.py:33-38 with a closed-form expectation."""
    packed = np.arange(256, dtype=np.uint8).reshape(16, 16)
    scales = np.full((16, 1), 127, dtype=np.uint8)
    got = om.decode_mxfp4(packed, scales)
    lut = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for r in range(16):
        for i in range(16):
            b = 16 * r + i
            for j, code in enumerate((b & 15, b >> 4)):
                want = -lut[code & 7] if code & 8 else lut[code & 7]
                g = got[r, 2 * i + j]
                assert g == want and math.copysign(1, g) == math.copysign(1, want)


def test_kat_all_scale_bytes_packed_0x22():
    """Restates tests/test_mxfp4_mlx.py:41-61: 0x22 is +1.0 in both nibbles, so every
    element of row s is 2**(s-127) in float32 (byte 0 subnormal, byte 255 +inf)."""
    packed = np.full((256, 16), 0x22, dtype=np.uint8)
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    got = om.decode_mxfp4(packed, scales)
    with np.errstate(over="ignore"):
        want = np.array([np.float32(math.ldexp(1.0, s - 127)) if s < 255 else np.float32(np.inf)
                         for s in range(256)], dtype=np.float32)
    assert np.array_equal(got, np.repeat(want[:, None], 32, axis=1))
    assert got[0, 0] > 0 and got[0, 0] < np.finfo(np.float32).tiny   # subnormal kept
    assert np.isinf(got[255]).all()


@pytest.mark.parametrize("k_pos", [0, 1, 2, 31, 32, 33, 63, 64, 127])
def test_layout_nibble_order_and_groups(k_pos):
    n, k = 3, 128
    packed = np.zeros((n, k // 2), dtype=np.uint8)
    scales = np.array([[120, 125, 130, 135]] * n, dtype=np.uint8)
    code = 0xB                                  # -1.5
    packed[1, k_pos // 2] = code << (4 * (k_pos & 1))
    got = om.decode_mxfp4(packed, scales)
    want = np.zeros((n, k), dtype=np.float32)
    want[1, k_pos] = -1.5 * 2.0 ** (int(scales[1, k_pos // 32]) - 127)
    assert np.array_equal(got, want)


def test_numpy_oracle_matches_c_restatement():
    native.build(force=False)
    rng = np.random.default_rng(123)
    packed = rng.integers(0, 256, size=(64, 512), dtype=np.uint8)
    scales = rng.integers(0, 256, size=(64, 32), dtype=np.uint8)   # every byte incl. 0/255
    a = om.decode_mxfp4(packed, scales)
    b = native.decode_f32(packed, scales)
    nan = np.isnan(a)
    assert np.array_equal(nan, np.isnan(b))
    assert np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan])


def test_f64_decode_is_the_widened_f32_decode():
    """The full-size oracles' float64 decode (C per-group table form) against the NumPy
    decode widened: every (code, scale byte) pair, with NaN from byte 255 x code 0/8, and a
    random tensor over every scale byte."""
    native.build(force=False)
    codes = np.arange(16, dtype=np.uint8)
    packed = np.zeros((256, 16), dtype=np.uint8)
    packed[:, :8] = (codes[0::2] | (codes[1::2] << 4))[None, :]
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    rng = np.random.default_rng(124)
    cases = [(packed, scales),
             (rng.integers(0, 256, size=(64, 512), dtype=np.uint8), rng.integers(0, 256, size=(64, 32), dtype=np.uint8))]
    for p, s in cases:
        a = om.decode_mxfp4(p, s).astype(np.float64)
        b = om.decode_mxfp4_f64(p, s)
        assert b.dtype == np.float64
        nan = np.isnan(a)
        assert np.array_equal(nan, np.isnan(b))
        assert np.array_equal(a.view(np.uint64)[~nan], b.view(np.uint64)[~nan])
    assert np.isinf(om.decode_mxfp4_f64(packed, scales)[255, 1])   # code 1 at byte 255


def test_matvec_onehot_returns_decoded_columns():
    rng = np.random.default_rng(5)
    packed, scales = om.random_mxfp4(rng, 48, 256)
    w = om.decode_mxfp4(packed, scales)
    for k in (0, 1, 31, 32, 200, 255):
        x = np.zeros(256, dtype=np.float32)
        x[k] = 1.0
        assert np.array_equal(om.matvec_f64(x, packed, scales), w[:, k].astype(np.float64))


@pytest.mark.parametrize("m", [1, 2, 4])
def test_matvec_f64_vs_reference_kernel_order(m):
    """Restates tests/test_mxfp4_kernel.py:42-54 with the C emulation of the Metal
    kernel's sequential fp32 FMA in place of the kernel: rel < 1e-6 vs fp64."""
    rng = np.random.default_rng(0)
    n, k = 128, 256
    packed = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = rng.integers(100, 140, size=(n, k // 32), dtype=np.uint8)
    x = rng.standard_normal((m, k)).astype(np.float32)
    want = om.matvec_f64(x, packed, scales)
    got = native.matvec_seqfma(x, packed, scales)
    assert om.normwise_rel(got, want) < 1e-6


def test_bf16_round_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(9)
    a = np.concatenate([
        rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 10000),
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.4e38, -3.4e38, 1e-40],
                 dtype=np.float32)]).astype(np.float32)
    want = torch.from_numpy(a).to(torch.bfloat16).float().numpy()
    assert np.array_equal(om.bf16_round(a).view(np.uint32), want.view(np.uint32))


def test_unfused_definition_equals_exact_for_bf16_inputs():
    """W is bf16-exact for normal scales, so for x already in bf16 the reference's unfused
    definition is the exact product; for fp32 x it differs only by x's bf16 rounding."""
    rng = np.random.default_rng(11)
    packed, scales = om.random_mxfp4(rng, 64, 512)
    x = om.bf16_round(rng.standard_normal((2, 512)).astype(np.float32))
    assert np.array_equal(om.matvec_unfused_f64(x, packed, scales), om.matvec_f64(x, packed, scales))
    xf = rng.standard_normal((2, 512)).astype(np.float32)
    rel = om.normwise_rel(om.matvec_unfused_f64(xf, packed, scales), om.matvec_f64(xf, packed, scales))
    assert 0 < rel < 2.0 ** -7


def test_encoder_roundtrip_error_bound():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((16, 256)).astype(np.float32)
    p, s = om.encode_mxfp4(w)
    back = om.decode_mxfp4(p, s)
    # group max lands in [4, 8) x scale: in-range error <= half the widest gap (4 -> 6),
    # values above 6 x scale clip to 6, so the bound is 2 x scale
    step = om.e8m0_to_f32(s).repeat(32, axis=1)
    assert np.all(np.abs(back - w) <= 2 * step)
    assert np.all((s >= 1) & (s <= 254))
