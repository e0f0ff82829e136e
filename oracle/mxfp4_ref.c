/*
 * Independent C restatement of the MXFP4 format, for the CPU oracle.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (and nothing in the product path).
 *
 * oracle_decode_f32  follows k3ref/weights.py:29-37 (float32 table value, sign flip,
 *                    ldexpf(1, b-127), one float32 multiply) using libm's ldexpf and a
 *                    branchy code path -- a different route from the NumPy oracle's
 *                    signed table + exponent-bit construction, so the two pin each other.
 * oracle_matvec_seqfma emulates the reference Metal kernel
 *                    (air_llm/kernels/metal/mxfp4_matvec.py:29-63): one accumulator per
 *                    output, K walked in ascending order, fmaf per element, scale built
 *                    as the float whose bit pattern is (byte << 23) -- so byte 0 gives
 *                    +0.0 there, exactly like the Metal source.
 * oracle_decode_f64  oracle_decode_f32 widened to float64, built from a per-group table of
 *                    the 16 float32 code values (fast enough for full-size oracles).
 *
 * Build: gcc -O2 -fPIC -shared -ffp-contract=off (no fast-math: subnormals matter).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static const float kMag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

static float code_value(unsigned code) {
    float m = kMag[code & 7u];
    return (code & 8u) ? -m : m;
}

void oracle_decode_f32(const uint8_t *packed, const uint8_t *scales,
                       int64_t n, int64_t k, float *out) {
    const int64_t kh = k / 2, g = k / 32;
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t i = 0; i < k; ++i) {
            uint8_t byte = packed[r * kh + i / 2];
            unsigned code = (i & 1) ? (unsigned)(byte >> 4) : (unsigned)(byte & 0x0F);
            float s = ldexpf(1.0f, (int)scales[r * g + i / 32] - 127);
            out[r * k + i] = code_value(code) * s;
        }
    }
}

static float bits_to_float(uint32_t b) {
    float f;
    memcpy(&f, &b, sizeof f);
    return f;
}

void oracle_matvec_seqfma(const float *x, const uint8_t *packed, const uint8_t *scales,
                          int64_t m, int64_t n, int64_t k, float *out) {
    const int64_t kh = k / 2, g = k / 32;
    for (int64_t t = 0; t < m; ++t) {
        for (int64_t r = 0; r < n; ++r) {
            float acc = 0.0f;
            for (int64_t kb = 0; kb < kh; ++kb) {
                uint8_t byte = packed[r * kh + kb];
                int64_t k0 = kb * 2;
                float s = bits_to_float((uint32_t)scales[r * g + k0 / 32] << 23);
                float v0 = code_value(byte & 0x0F) * s;
                float v1 = code_value(byte >> 4) * s;
                acc = fmaf(x[t * k + k0], v0, acc);
                acc = fmaf(x[t * k + k0 + 1], v1, acc);
            }
            out[t * n + r] = acc;
        }
    }
}

/* oracle_decode_f64: the float64 widening of oracle_decode_f32, bit for bit, for the
 * full-size oracles.  Per row group the 16 code values are formed once exactly as
 * oracle_decode_f32 forms each element (code value times ldexpf(1, b-127) in float32,
 * so byte 255 gives inf/NaN and bytes 253..254 overflow as there), then widened; each
 * packed byte then reads two of them from that table. */
void oracle_decode_f64(const uint8_t *packed, const uint8_t *scales,
                       int64_t n, int64_t k, double *out) {
    const int64_t kh = k / 2, g = k / 32;
    double vals[16];
    for (int64_t r = 0; r < n; ++r) {
        for (int64_t j = 0; j < g; ++j) {
            const float s = ldexpf(1.0f, (int)scales[r * g + j] - 127);
            for (unsigned c = 0; c < 16; ++c) vals[c] = (double)(code_value(c) * s);
            const uint8_t *p = packed + r * kh + j * 16;
            double *o = out + r * k + j * 32;
            for (int i = 0; i < 16; ++i) {
                o[2 * i] = vals[p[i] & 0x0F];
                o[2 * i + 1] = vals[p[i] >> 4];
            }
        }
    }
}
