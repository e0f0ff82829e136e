"""MXFP4 oracle (test infrastructure only; see ``oracle/__init__.py``).

Format (``air_llm/models/kimi_k3/mxfp4.py:3-11``, ``k3ref/weights.py:26-37``):

* ``packed`` is ``uint8 [N, K/2]``; element ``2i`` of a row is the LOW nibble of byte
  ``i`` and element ``2i+1`` the HIGH nibble.
* a nibble is an E2M1 code: bit 3 is the sign, bits 0-2 index
  ``{0, 0.5, 1, 1.5, 2, 3, 4, 6}``.  Code 8 is negative zero.
* ``scales`` is ``uint8 [N, K/32]``; byte ``b`` is the E8M0 power of two ``2**(b-127)``
  applied to the 32 consecutive elements ``32j .. 32j+31`` of the row.

The reference computes the decode in float32: a float32 table lookup, a sign flip, an
``ldexp`` of 1.0f by ``b-127`` (so byte 0 is the subnormal ``2**-127`` and byte 255
overflows to ``+inf``), and one float32 multiply.  ``decode_mxfp4`` below reaches the same
float32 values through a signed 16-entry table and an exponent-field bit construction of
the scale.

Pinning (``tests/test_oracle_mxfp4.py``):

* the 16 x 256 (code, scale byte) truth table against exact rational arithmetic
  (``fractions.Fraction``) rounded to float32 with IEEE overflow / invalid rules;
* the two known-answer tests of ``tests/test_mxfp4_mlx.py:33-61`` (every packed byte at
  scale 127; every scale byte with packed ``0x22``) against closed-form expectations;
* nibble order / group placement by planting single codes at chosen positions;
* bit-identity with the independent C restatement in ``oracle/mxfp4_ref.c``;
* the fp64 matvec against one-hot inputs (which must return decoded columns exactly) and
  against the C emulation of the reference Metal kernel's sequential fp32 FMA order.
"""
from __future__ import annotations

import numpy as np

GROUP = 32

# Unsigned E2M1 magnitudes, indexed by code & 7.
E2M1_MAG = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)

# All 16 signed codes.  Negating the float32 magnitudes keeps code 8 as -0.0, which is
# what the reference's ``np.where(sign, -mag, mag)`` produces.
FP4_VALUES = np.concatenate([E2M1_MAG, -E2M1_MAG]).astype(np.float32)


def e8m0_to_f32(scales: np.ndarray) -> np.ndarray:
    """E8M0 byte -> float32 ``2**(b-127)`` with the reference's float32 ldexp semantics.

    Bytes 1..254 are normal numbers whose exponent field is the byte itself.  Byte 0 is
    the subnormal ``2**-127`` (bit pattern 0x00400000); byte 255 is ``+inf``
    (``ldexp(1.0f, 128)`` overflows), i.e. bit pattern 0x7F800000 == 255 << 23.
    """
    s = np.asarray(scales, dtype=np.uint8)
    bits = s.astype(np.uint32) << 23
    bits = np.where(s == 0, np.uint32(0x00400000), bits).astype(np.uint32)
    return bits.view(np.float32)


def unpack_codes(packed: np.ndarray) -> np.ndarray:
    """uint8 [N, K/2] -> uint8 codes [N, K], low nibble first."""
    p = np.asarray(packed, dtype=np.uint8)
    return np.stack([p & 0x0F, p >> 4], axis=-1).reshape(p.shape[0], p.shape[1] * 2)


def decode_mxfp4(packed: np.ndarray, scales: np.ndarray, group_size: int = GROUP) -> np.ndarray:
    """Bit-exact float32 decode, following ``k3ref/weights.py:29-37``."""
    packed = np.asarray(packed, dtype=np.uint8)
    scales = np.asarray(scales, dtype=np.uint8)
    n, kh = packed.shape
    k = kh * 2
    if k % group_size or scales.shape != (n, k // group_size):
        raise ValueError(f"scales shape {scales.shape} does not match packed {packed.shape}")
    vals = FP4_VALUES[unpack_codes(packed)].reshape(n, k // group_size, group_size)
    with np.errstate(invalid="ignore", over="ignore"):
        out = vals * e8m0_to_f32(scales)[:, :, None]
    return out.reshape(n, k).astype(np.float32, copy=False)


def decode_mxfp4_f64(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """``decode_mxfp4`` widened to float64, for the full-size oracles: the C restatement's
    per-group table form (``oracle/mxfp4_ref.c``, ``oracle_decode_f64``) when its library is
    built, else the NumPy decode widened.  The two are bit-identical (pinned in
    ``tests/test_oracle_mxfp4.py``); the C form is about 15x faster and releases the GIL."""
    try:
        from . import native
        native.load()
    except OSError:
        return decode_mxfp4(packed, scales).astype(np.float64)
    return native.decode_f64(packed, scales)


def matvec_f64(x: np.ndarray, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """``x @ W.T`` in float64 on the exactly decoded W -- the oracle of
    ``tests/test_mxfp4_kernel.py:48-54``.  x: [M, K] or [K]."""
    w = decode_mxfp4(packed, scales).astype(np.float64)
    return np.asarray(x, dtype=np.float64) @ w.T


def bf16_round(a: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32.  NaN stays NaN."""
    a = np.asarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = (r.astype(np.uint32) << 16).view(np.float32)
    return np.where(np.isnan(a), a, out).astype(np.float32)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bfloat16 bit patterns (ties to even)."""
    return (bf16_round(a).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def matvec_unfused_f64(x: np.ndarray, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """The reference's own dequant-then-matmul (``mxfp4.py:84-92``): x rounded to bf16,
    W decoded to bf16 (exact for normal scales), products accumulated -- here in fp64,
    i.e. the exact value of the bf16 x bf16 contraction that the reference accumulates in
    fp32."""
    w = decode_mxfp4(packed, scales)
    return bf16_round(np.asarray(x, dtype=np.float32)).astype(np.float64) @ \
        bf16_round(w).astype(np.float64).T


def normwise_rel(got: np.ndarray, want: np.ndarray) -> float:
    """``max|got - want| / max|want|`` -- the metric of ``tests/test_mxfp4_kernel.py:53``."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.abs(got - want).max() / max(float(np.abs(want).max()), 1e-30))


# --------------------------------------------------------------------- synthetic data

def random_mxfp4(rng: np.random.Generator, n: int, k: int, lo: int = 118, hi: int = 130):
    """Random packed bytes (all 16 codes, including -0) and E8M0 bytes uniform in
    [lo, hi] inclusive -- the synthetic weights of the benchmark configurations."""
    packed = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scales = rng.integers(lo, hi + 1, size=(n, k // GROUP), dtype=np.uint8)
    return packed, scales


def encode_mxfp4(w: np.ndarray, group_size: int = GROUP):
    """float -> (packed, scales): a realistic encoder for fixtures.

    The E8M0 exponent puts the group's absolute maximum in [4, 8) (the OCP MX rule
    ``floor(log2(amax)) - emax(E2M1)``), then every element goes to the nearest E2M1
    magnitude (ties to the lower code).  The format contract this satisfies is the one
    ``decode_mxfp4`` reads; the encoder itself is not on the hot path.
    """
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    g = w.reshape(n, k // group_size, group_size)
    amax = np.abs(g).max(axis=-1)
    exp = np.floor(np.log2(np.where(amax > 0, amax, 1.0))).astype(np.int32) - 2
    sbyte = np.clip(exp + 127, 1, 254).astype(np.uint8)
    q = g / e8m0_to_f32(sbyte)[:, :, None]
    mag_idx = np.abs(np.abs(q)[..., None] - E2M1_MAG).argmin(axis=-1).astype(np.uint8)
    codes = (mag_idx | (np.signbit(q).astype(np.uint8) << 3)).reshape(n, k)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8)
    return packed, sbyte
