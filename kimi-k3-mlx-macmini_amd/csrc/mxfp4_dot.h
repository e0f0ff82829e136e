// Per-group MXFP4 dot products and the LDS activation tile shared by the GEMV, expert
// and MoE-layer kernels.
#pragma once

#include <type_traits>

#include "k3_common.h"

namespace k3 {

template <typename XT>
struct XTile;
template <>
struct XTile<uint16_t> {  // bf16 activations: a group is 64 bytes = 4 chunks
    static constexpr int kChunks = 4;
    __device__ static int slot(int g, int q) { return g * 4 + (q ^ ((g >> 1) & 3)); }
};
template <>
struct XTile<float> {  // fp32 activations: a group is 128 bytes = 8 chunks
    static constexpr int kChunks = 8;
    __device__ static int slot(int g, int q) { return g * 8 + (q ^ (g & 7)); }
};

// 32-element dot of one packed group (16 bytes) with bf16 activations (4 chunks).
__device__ __forceinline__ float group_dot(const uint4 w, const uint4 *xc) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    float p0 = 0.f, p1 = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint4 c = xc[d];
        const uint32_t xw[4] = {c.x, c.y, c.z, c.w};
        p0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[d], 1.0f, 0),
                                             __builtin_bit_cast(bf16x2, xw[0]), p0, false);
        p1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[d], 1.0f, 1),
                                             __builtin_bit_cast(bf16x2, xw[1]), p1, false);
        p0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[d], 1.0f, 2),
                                             __builtin_bit_cast(bf16x2, xw[2]), p0, false);
        p1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[d], 1.0f, 3),
                                             __builtin_bit_cast(bf16x2, xw[3]), p1, false);
    }
    return p0 + p1;
}

// Dot of ND packed dwords (8 * ND elements) with fp32 activations (2 * ND chunks of 4 floats).
template <int ND>
__device__ __forceinline__ float piece_dot(const uint32_t (&wd)[ND], const float4 *xc) {
    float p0 = 0.f, p1 = 0.f;
#pragma unroll
    for (int d = 0; d < ND; ++d) {
        const float4 a = xc[2 * d], b = xc[2 * d + 1];
        f32x2 w0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd[d], 1.0f, 0);
        f32x2 w1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd[d], 1.0f, 1);
        f32x2 w2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd[d], 1.0f, 2);
        f32x2 w3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(wd[d], 1.0f, 3);
        p0 = fmaf(a.x, w0.x, p0);
        p1 = fmaf(a.y, w0.y, p1);
        p0 = fmaf(a.z, w1.x, p0);
        p1 = fmaf(a.w, w1.y, p1);
        p0 = fmaf(b.x, w2.x, p0);
        p1 = fmaf(b.y, w2.y, p1);
        p0 = fmaf(b.z, w3.x, p0);
        p1 = fmaf(b.w, w3.y, p1);
    }
    return p0 + p1;
}

// 32-element dot of one packed group with fp32 activations (8 chunks of 4 floats).
__device__ __forceinline__ float group_dot(const uint4 w, const float4 *xc) {
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    return piece_dot<4>(wd, xc);
}

template <typename XT>
using XChunk = typename std::conditional<std::is_same<XT, float>::value, float4, uint4>::type;

// Stage n_chunks 16-byte activation chunks of one token into the swizzled LDS tile.
template <typename XT>
__device__ __forceinline__ void stage_x_tile(uint4 *xs, const void *x, int n_chunks) {
    constexpr int CPG = XTile<XT>::kChunks;
    const uint4 *src = static_cast<const uint4 *>(x);
    for (int c = threadIdx.x; c < n_chunks; c += blockDim.x) xs[XTile<XT>::slot(c / CPG, c % CPG)] = src[c];
}

}  // namespace k3
