// Shared device/host helpers for the k3hip kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/k3hip.h"

namespace k3 {

constexpr int kWave = 64;

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------- error reporting
int set_error(int code, const char *fmt, ...);
int check_hip(hipError_t e, const char *what);

inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The absorbed MLA decode core behind k3_mla_decode_absorbed(_f32), with an optional output
// gate: gate [H, v_dim] fp32 logits (null: none) multiply o by sigmoid(gate) as it is
// written.  cache_dtype: K3_BF16 or K3_F32 rows of lat and rot.
int mla_decode_core(const void *q_nope, const void *q_rot, int64_t ld_q, int64_t ld_q_rot, int q_dtype,
                    const void *w_uk, const void *w_uv, const void *lat, int64_t ld_lat, const void *rot,
                    int64_t ld_rot, int64_t T, int64_t H, int64_t kv_lora_rank, int64_t rope_dim, int64_t nope_dim,
                    int64_t v_dim, float scale, void *out, int out_dtype, int64_t ld_out, const float *gate,
                    void *workspace, int64_t workspace_bytes, void *stream, int cache_dtype = K3_BF16);

// ---------------------------------------------------------------- bf16 <-> f32
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
// Round-to-nearest-even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// E8M0 byte -> float32 2^(b-127).  Byte 0 is the subnormal 2^-127, byte 255 is +inf
// (the float32 ldexp semantics of k3ref/weights.py:36).
__device__ __forceinline__ float e8m0_to_f32(uint32_t b) {
    return __uint_as_float(b == 0u ? 0x00400000u : (b << 23));
}

// ---------------------------------------------------------------- wave reductions
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp_or_zero(float v) {
    // lanes whose row is masked off (or whose source is invalid) read 0
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK,
                                                      BANK_MASK, true));
}

// Full wave64 sum; the total lands in lane 63.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
    v += dpp_or_zero<0xb1>(v);         // quad_perm [1,0,3,2]
    v += dpp_or_zero<0x4e>(v);         // quad_perm [2,3,0,1]
    v += dpp_or_zero<0x141>(v);        // row_half_mirror
    v += dpp_or_zero<0x140>(v);        // row_mirror  -> every lane holds its row's sum
    v += dpp_or_zero<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
    v += dpp_or_zero<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
    return v;
}

// Full wave64 sum broadcast to every lane.
__device__ __forceinline__ float wave_sum_all(float v) {
    v = wave_sum_to_lane63(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Value of lane `row * 16` after a row-wide reduction: the four row results are combined
// through v_readlane (SGPRs), so no step waits on an LDS round trip (ds_bpermute).
__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Full wave64 max broadcast to every lane: DPP inside each 16-lane row, then the 4 rows.
__device__ __forceinline__ float wave_max_all(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false)));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------- buffer loads
// Raw buffer resource over [base, base + bytes): loads whose byte offset falls outside
// return zeros, which lets tails and invalid rows load without branches.
constexpr uint32_t kOobOffset = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// The same load with the non-temporal hint (the nt bit of the cache policy), for weight rows
// that a launch streams once: measured on the batch-1 expert step 9.4 -> 9.2 us, the
// 384-expert layer's four-token step 171 -> 161.5 us, K3's layer 128 -> 121-123 us, the KDA
// step 175 -> 154 us.  The weights' E8M0 scale bytes load with the same hint (aux 2 on
// their byte and dword loads): expert step 2560 -> 2630 GB/s, batch-1 GEMV 3.98 -> 3.84 us.
// Inputs that several blocks stage (x, act, norm weights) keep the default policy: the hint
// on every load made the expert step 20% slower.  The grouped prefill's weight tiles (read
// once per token tile of an expert) and the MLA cache rows (read by the four head-group
// blocks of a split) keep it too: with the hint, 4.65 -> 5.18 ms and no gain.
__device__ __forceinline__ uint4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

}  // namespace k3
