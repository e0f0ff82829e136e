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

// E8M0 bytes staged per wave.  A wave needs the scale bytes of NS row slices (slice s: SW
// consecutive bytes from byte offset off_s of a scale matrix).  One byte load per (row, group)
// makes a 64-byte request per wave instruction, as many instructions as weight loads; instead
// lane l < NS * kCPR loads the 16-byte chunk l % kCPR of slice l / kCPR (chunks start at
// off_s rounded down to 16, hence one extra chunk), the wave stores its chunks in its own LDS
// area, and every lane reads its bytes there (consecutive lanes read consecutive bytes).
template <int SW>
struct ScaleStage {
    static constexpr int kCPR = SW / 16 + 1;  // 16-byte chunks per slice
    __device__ static int slice_of(int lane) { return lane / kCPR; }
    // byte offset (in the scale matrix) of the chunk `lane` loads for a slice at `off`
    __device__ static uint32_t chunk_off(uint32_t off, int lane) { return (off & ~15u) + 16u * (lane % kCPR); }
    // byte offset, in the wave's LDS area, of byte j of slice s (slice at `off`)
    __device__ static uint32_t at(int s, uint32_t off, int j) { return s * (kCPR * 16) + (off & 15u) + j; }
};

// Buffer resource over a scale matrix of `bytes` bytes whose base is rounded down to 16, so
// that every chunk load is 16-byte aligned; `mis` (0..15) is added to every byte offset.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_scale_rsrc(const void *scales, uint32_t bytes, uint32_t &mis) {
    mis = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(scales) & 15u);
    return make_rsrc(static_cast<const uint8_t *>(scales) - mis, bytes + mis);
}

// Stage n_chunks 16-byte activation chunks of one token into the swizzled LDS tile.
template <typename XT>
__device__ __forceinline__ void stage_x_tile(uint4 *xs, const void *x, int n_chunks) {
    constexpr int CPG = XTile<XT>::kChunks;
    const uint4 *src = static_cast<const uint4 *>(x);
    for (int c = threadIdx.x; c < n_chunks; c += blockDim.x) xs[XTile<XT>::slot(c / CPG, c % CPG)] = src[c];
}

}  // namespace k3
