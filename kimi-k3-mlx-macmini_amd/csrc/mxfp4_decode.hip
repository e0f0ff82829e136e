// Bit-exact MXFP4 -> fp32 / bf16 dequantisation and the E8M0 range guard.
//
// Semantics follow k3ref/weights.py:29-37 (float32 table value, sign, ldexp(1, b-127),
// one float32 multiply), so byte 0 decodes through the subnormal 2^-127 and byte 255
// through +inf.  The product of an E2M1 magnitude (<= 2 significant bits) and a power of
// two is exact whenever it does not overflow, so the fp32 result equals the reference's
// bit for bit and the bf16 result is that fp32 value truncated (exact: the low 16 bits
// are zero, NaN stays NaN).
#include "k3_common.h"

namespace k3 {
namespace {

// E2M1 code -> float32 bit pattern: 0, 0.5, 1, 1.5, 2, 3, 4, 6 with bit 3 as the sign.
__device__ __forceinline__ uint32_t e2m1_bits(uint32_t c) {
    const uint32_t m3 = c & 7u;
    const uint32_t mag = m3 < 2u ? (m3 ? 0x3F000000u : 0u)
                                 : (((126u + (m3 >> 1)) << 23) | ((m3 & 1u) << 22));
    return mag | ((c & 8u) << 28);
}

// One thread per 4 packed bytes (8 elements).  Packed and scales are contiguous, so the
// flat index of the 4-byte word determines its row, and its group is word / 4.
template <bool BF16_OUT>
__global__ __launch_bounds__(256) void decode_kernel(const uint32_t *__restrict__ packed,
                                                     const uint8_t *__restrict__ scales,
                                                     void *__restrict__ out, int64_t n_words) {
    const int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (w >= n_words) return;
    const uint32_t bits = packed[w];
    const float s = e8m0_to_f32(scales[w >> 2]);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(e2m1_bits((bits >> (4 * i)) & 15u)) * s;
    if constexpr (BF16_OUT) {
        uint4 o;
        o.x = (__float_as_uint(v[0]) >> 16) | (__float_as_uint(v[1]) & 0xffff0000u);
        o.y = (__float_as_uint(v[2]) >> 16) | (__float_as_uint(v[3]) & 0xffff0000u);
        o.z = (__float_as_uint(v[4]) >> 16) | (__float_as_uint(v[5]) & 0xffff0000u);
        o.w = (__float_as_uint(v[6]) >> 16) | (__float_as_uint(v[7]) & 0xffff0000u);
        reinterpret_cast<uint4 *>(out)[w] = o;
    } else {
        float4 *o = reinterpret_cast<float4 *>(out) + 2 * w;
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
}

__global__ void minmax_init(int32_t *mm) {
    mm[0] = 255;
    mm[1] = 0;
}

__global__ __launch_bounds__(256) void minmax_kernel(const uint8_t *__restrict__ s, int64_t n,
                                                     int32_t *__restrict__ mm) {
    int lo = 255, hi = 0;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int b = s[i];
        lo = min(lo, b);
        hi = max(hi, b);
    }
    for (int off = 32; off > 0; off >>= 1) {
        lo = min(lo, __shfl_xor(lo, off, kWave));
        hi = max(hi, __shfl_xor(hi, off, kWave));
    }
    if ((threadIdx.x & (kWave - 1)) == 0) {
        atomicMin(mm, lo);
        atomicMax(mm + 1, hi);
    }
}

}  // namespace
}  // namespace k3

using namespace k3;

extern "C" int k3_mxfp4_decode(const void *packed, const void *scales, void *out, int out_dtype,
                               int64_t N, int64_t K, void *stream) {
    if (!packed || !scales || !out) return set_error(K3_ERR_NULL, "k3_mxfp4_decode: null pointer");
    if (N < 0 || K < 0 || K % 32 != 0)
        return set_error(K3_ERR_SHAPE, "k3_mxfp4_decode: K=%lld must be a multiple of 32",
                         (long long)K);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "k3_mxfp4_decode: out_dtype %d", out_dtype);
    if ((reinterpret_cast<uintptr_t>(packed) & 3u) || !aligned16(out))
        return set_error(K3_ERR_ALIGN, "k3_mxfp4_decode: packed must be 4-byte and out 16-byte aligned");
    const int64_t n_words = N * K / 8;
    if (n_words == 0) return K3_OK;
    const dim3 grid(static_cast<unsigned>(cdiv(n_words, 256)));
    auto st = static_cast<hipStream_t>(stream);
    if (out_dtype == K3_BF16)
        decode_kernel<true><<<grid, 256, 0, st>>>(static_cast<const uint32_t *>(packed),
                                                  static_cast<const uint8_t *>(scales), out, n_words);
    else
        decode_kernel<false><<<grid, 256, 0, st>>>(static_cast<const uint32_t *>(packed),
                                                   static_cast<const uint8_t *>(scales), out, n_words);
    return check_hip(hipGetLastError(), "k3_mxfp4_decode launch");
}

extern "C" int k3_scale_minmax(const void *scales, int64_t n, int32_t *minmax, void *stream) {
    if (!scales || !minmax) return set_error(K3_ERR_NULL, "k3_scale_minmax: null pointer");
    if (n < 0) return set_error(K3_ERR_SHAPE, "k3_scale_minmax: n < 0");
    auto st = static_cast<hipStream_t>(stream);
    minmax_init<<<1, 1, 0, st>>>(minmax);
    if (n > 0) {
        const int64_t blocks = std::min<int64_t>(cdiv(n, 256 * 16), 1024);
        minmax_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, st>>>(
            static_cast<const uint8_t *>(scales), n, minmax);
    }
    return check_hip(hipGetLastError(), "k3_scale_minmax launch");
}
