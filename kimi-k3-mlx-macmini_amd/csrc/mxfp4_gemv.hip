// Fused MXFP4 matvec / small-M matmul for gfx950 (the batch-1 expert GEMV).
//
// Replaces the reference Metal kernel (air_llm/kernels/metal/mxfp4_matvec.py:29-63), which
// runs one thread per output and walks a packed row byte by byte.  Here:
//
//   * a wave owns RPW weight rows; its 64 lanes sweep the row's 32-element groups, lane l
//     taking groups l, l+64, ... so every 128-bit load of packed nibbles is part of a
//     contiguous 1 KiB wave-wide read (one group = 16 packed bytes = one E8M0 scale);
//   * the block's scale rows (contiguous in [N, K/32]) are staged in LDS with 128-bit
//     loads, and the activation tokens are staged in LDS once per block, in a swizzled
//     16-byte-chunk order so the per-lane group reads do not collide on LDS banks;
//   * nibbles become bf16 pairs (bf16 activations: v_cvt_scalef32_pk_bf16_fp4 then
//     v_dot2_f32_bf16) or fp32 pairs (fp32 activations: v_cvt_scalef32_pk_f32_fp4 then
//     fp32 FMA); each group's partial sum is scaled once by its power-of-two E8M0 scale
//     (exact) and accumulated in fp32;
//   * the next sweep's weights are loaded before the current one is consumed, and the
//     per-lane partials are summed with a DPP wave reduction.
//
// Numerics: weights are exact (E2M1 x 2^e), products of bf16/fp32 activations with them
// are exact in fp32, accumulation is fp32 -- the same arithmetic class as the reference
// fused kernel, with a different (grouped, then tree) summation order.
#include "k3_common.h"
#include "mxfp4_dot.h"
#include "mxfp4_gemv.h"

namespace k3 {

template <typename XT, int RPW, int GPL, int MT>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    extern __shared__ uint4 smem[];
    constexpr int CPG = XTile<XT>::kChunks;
    constexpr int BR = 4 * RPW;
    constexpr int XREG = MT == 1 ? 8 : 2;  // activation chunks staged per thread in one batch
    const int G = static_cast<int>(a.K >> 5);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BR;
    const int rows_here = static_cast<int>(min<int64_t>(BR, a.N - n0));
    const uint32_t row_bytes = static_cast<uint32_t>(a.K >> 1);

    uint4 *xs = smem;
    uint8_t *ss = reinterpret_cast<uint8_t *>(smem + MT * G * CPG);

    // 1. small loads first: this block's scale rows and the first batch of activation
    //    chunks (L2-resident after the first block), so their wait does not include the
    //    weight stream issued right after them
    const auto srsrc = make_rsrc(static_cast<const uint8_t *>(a.scales) + n0 * G,
                                 static_cast<uint32_t>(rows_here * G));
    const int schunks = (rows_here * G + 15) >> 4;
    uint4 sreg[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = threadIdx.x + 256 * i;
        sreg[i] = buf_load16(srsrc, (a.scales_vec && c < schunks) ? static_cast<uint32_t>(c) * 16u : kOobOffset);
    }

    const int xchunks = G * CPG;
    const int xbatch = min(xchunks, 256 * XREG);
    uint4 xreg[MT][XREG];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const auto xr = make_rsrc(static_cast<const XT *>(a.x) + m * a.ldx,
                                  m < a.M ? static_cast<uint32_t>(xchunks * 16) : 0u);
#pragma unroll
        for (int i = 0; i < XREG; ++i) {
            const int c = threadIdx.x + 256 * i;
            xreg[m][i] = buf_load16(xr, c < xbatch ? static_cast<uint32_t>(c) * 16u : kOobOffset);
        }
    }

    // 2. the first sweep of weights; rows past N and groups past G read zeros
    const auto wrsrc = make_rsrc(a.packed, static_cast<uint32_t>(a.N * row_bytes));
    uint4 wreg[RPW][GPL];
    auto load_sweep = [&](int gs) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int64_t n = n0 + wave * RPW + r;
#pragma unroll
            for (int u = 0; u < GPL; ++u) {
                const int g = gs + u * kWave + lane;
                const uint32_t off = (n < a.N && g < G)
                                         ? static_cast<uint32_t>(n) * row_bytes + static_cast<uint32_t>(g) * 16u
                                         : kOobOffset;
                wreg[r][u] = buf_load16(wrsrc, off);
            }
        }
    };
    load_sweep(0);

    // 3. stage into LDS (activations in swizzled chunk order)
    if (a.scales_vec) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = threadIdx.x + 256 * i;
            if (c < schunks) reinterpret_cast<uint4 *>(ss)[c] = sreg[i];
        }
        for (int c = 512 + threadIdx.x; c < schunks; c += 256)
            reinterpret_cast<uint4 *>(ss)[c] = buf_load16(srsrc, static_cast<uint32_t>(c) * 16u);
    } else {
        const uint8_t *src = static_cast<const uint8_t *>(a.scales) + n0 * G;
        for (int c = threadIdx.x; c < rows_here * G; c += 256) ss[c] = src[c];
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int i = 0; i < XREG; ++i) {
            const int c = threadIdx.x + 256 * i;
            if (m < a.M && c < xbatch) xs[m * xchunks + XTile<XT>::slot(c / CPG, c % CPG)] = xreg[m][i];
        }
        if (m < a.M && xchunks > xbatch) {  // long rows: the rest, one chunk at a time
            const uint4 *src = reinterpret_cast<const uint4 *>(static_cast<const XT *>(a.x) + m * a.ldx);
            for (int c = xbatch + threadIdx.x; c < xchunks; c += 256)
                xs[m * xchunks + XTile<XT>::slot(c / CPG, c % CPG)] = src[c];
        }
    }
    __syncthreads();

    // 4. sweeps over K: prefetch the next sweep, consume the current one
    float acc[MT][RPW];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[m][r] = 0.f;

    for (int gs = 0; gs < G; gs += kWave * GPL) {
        uint4 cur[RPW][GPL];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int u = 0; u < GPL; ++u) cur[r][u] = wreg[r][u];
        if (gs + kWave * GPL < G) load_sweep(gs + kWave * GPL);
#pragma unroll
        for (int u = 0; u < GPL; ++u) {
            const int g = gs + u * kWave + lane;
            if (g < G) {
                float sc[RPW];
#pragma unroll
                for (int r = 0; r < RPW; ++r) sc[r] = e8m0_to_f32(ss[(wave * RPW + r) * G + g]);
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    if (m < a.M) {
                        XChunk<XT> xc[CPG];
#pragma unroll
                        for (int q = 0; q < CPG; ++q)
                            xc[q] = reinterpret_cast<const XChunk<XT> *>(xs)[m * xchunks + XTile<XT>::slot(g, q)];
#pragma unroll
                        for (int r = 0; r < RPW; ++r) acc[m][r] = fmaf(group_dot(cur[r][u], xc), sc[r], acc[m][r]);
                    }
                }
            }
        }
    }

    // 5. wave reduction and store (lane 63 holds each total)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const float t = wave_sum_to_lane63(acc[m][r]);
            const int64_t n = n0 + wave * RPW + r;
            if (lane == 63 && m < a.M && n < a.N) {
                if (a.out_bf16)
                    static_cast<uint16_t *>(a.out)[m * a.ldo + n] = f32_to_bf16(t);
                else
                    static_cast<float *>(a.out)[m * a.ldo + n] = t;
            }
        }
    }
}

template <typename XT, int RPW, int GPL, int MT>
static int launch_one(const GemvArgs &a, hipStream_t st) {
    constexpr int CPG = XTile<XT>::kChunks;
    const int G = static_cast<int>(a.K >> 5);
    const size_t lds = static_cast<size_t>(MT) * G * CPG * 16 + ((4 * RPW * G + 15) & ~15);
    if (lds > kGemvMaxLds)
        return set_error(K3_ERR_SHAPE, "mxfp4 matvec: K=%lld needs %zu bytes of LDS (max %zu)",
                         (long long)a.K, lds, kGemvMaxLds);
    if (lds > 64 * 1024) {  // above the default dynamic-LDS limit: opt in (gfx950 has 160 KiB)
        int rc = check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_kernel<XT, RPW, GPL, MT>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)),
                           "mxfp4 matvec: raise LDS limit");
        if (rc) return rc;
    }
    const dim3 grid(static_cast<unsigned>(cdiv(a.N, 4 * RPW)));
    gemv_kernel<XT, RPW, GPL, MT><<<grid, 256, lds, st>>>(a);
    return check_hip(hipGetLastError(), "mxfp4 matvec launch");
}

template <typename XT, int MT>
static int dispatch_cfg(const GemvArgs &a, int rpw, int gpl, hipStream_t st) {
#define K3_CFG(R, U) \
    if (rpw == R && gpl == U) return launch_one<XT, R, U, MT>(a, st);
    K3_CFG(1, 4) K3_CFG(2, 4) K3_CFG(1, 2) K3_CFG(2, 2) K3_CFG(4, 2) K3_CFG(1, 1) K3_CFG(2, 1)
    K3_CFG(4, 1)
    if constexpr (MT == 1) { K3_CFG(8, 1) }
#undef K3_CFG
    return set_error(K3_ERR_SHAPE, "mxfp4 matvec: no kernel for rpw=%d gpl=%d", rpw, gpl);
}

// Default launch shape: cover K in at most one or two sweeps and keep >= ~2 blocks per CU.
void gemv_default_cfg(int64_t N, int64_t K, int *rpw, int *gpl) {
    const int64_t G = K / 32;
    *gpl = G > 128 ? 4 : (G > 64 ? 2 : 1);
    if (*gpl == 1)
        *rpw = N >= 16 * 512 ? 8 : (N >= 8 * 512 ? 4 : (N >= 4 * 256 ? 2 : 1));
    else if (*gpl == 2)
        *rpw = N >= 8 * 512 ? 4 : (N >= 4 * 512 ? 2 : 1);
    else
        *rpw = N >= 4 * 2 * 512 ? 2 : 1;
    if (*rpw == 8 && *gpl != 1) *rpw = 4;
    if (*rpw == 4 && *gpl == 4) *rpw = 2;
}

int gemv_launch(const GemvArgs &a, int rpw, int gpl, hipStream_t st) {
    if (a.x_bf16) {
        if (a.M == 1) return dispatch_cfg<uint16_t, 1>(a, rpw, gpl, st);
        return dispatch_cfg<uint16_t, 4>(a, rpw, gpl, st);
    }
    if (a.M == 1) return dispatch_cfg<float, 1>(a, rpw, gpl, st);
    return dispatch_cfg<float, 4>(a, rpw, gpl, st);
}

int gemv_validate(const void *x, int x_dtype, const void *packed, const void *scales,
                  const void *out, int out_dtype, int64_t M, int64_t N, int64_t K) {
    if ((M > 0 && N > 0) && (!x || !packed || !scales || !out))
        return set_error(K3_ERR_NULL, "mxfp4 matvec: null pointer");
    if (x_dtype != K3_F32 && x_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "mxfp4 matvec: x_dtype %d", x_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "mxfp4 matvec: out_dtype %d", out_dtype);
    if (M < 0 || N < 0 || K <= 0 || K % 32 != 0 || K >= (1ll << 31))
        return set_error(K3_ERR_SHAPE, "mxfp4 matvec: K=%lld must be a positive multiple of 32",
                         (long long)K);
    if (M == 0 || N == 0) return K3_OK;
    if (!aligned16(x) || !aligned16(packed))
        return set_error(K3_ERR_ALIGN, "mxfp4 matvec: x and packed must be 16-byte aligned");
    if (N * (K / 2) >= (1ll << 31))
        return set_error(K3_ERR_SHAPE, "mxfp4 matvec: one weight matrix must be < 2 GiB packed");
    return K3_OK;
}

}  // namespace k3

using namespace k3;

static int matvec_impl(const void *x, int x_dtype, const void *packed, const void *scales, void *out,
                       int out_dtype, int64_t M, int64_t N, int64_t K, int rpw, int gpl,
                       void *stream) {
    int rc = gemv_validate(x, x_dtype, packed, scales, out, out_dtype, M, N, K);
    if (rc) return rc;
    if (M == 0 || N == 0) return K3_OK;
    if (rpw <= 0 || gpl <= 0) gemv_default_cfg(N, K, &rpw, &gpl);
    if (M > 1 && rpw == 8) rpw = 4;
    const size_t xsz = x_dtype == K3_BF16 ? 2 : 4;
    const size_t osz = out_dtype == K3_BF16 ? 2 : 4;
    auto st = static_cast<hipStream_t>(stream);
    for (int64_t m0 = 0; m0 < M; m0 += 4) {  // token tiles of up to 4 share one weight pass
        GemvArgs a{};
        a.x = static_cast<const char *>(x) + m0 * K * xsz;
        a.ldx = K;
        a.packed = packed;
        a.scales = scales;
        a.out = static_cast<char *>(out) + m0 * N * osz;
        a.ldo = N;
        a.M = static_cast<int>(std::min<int64_t>(4, M - m0));
        a.N = N;
        a.K = K;
        a.x_bf16 = x_dtype == K3_BF16;
        a.out_bf16 = out_dtype == K3_BF16;
        a.scales_vec = ((K / 32) % 16 == 0) && aligned16(scales);
        rc = gemv_launch(a, rpw, gpl, st);
        if (rc) return rc;
    }
    return K3_OK;
}

extern "C" int k3_mxfp4_matvec(const void *x, int x_dtype, const void *packed, const void *scales,
                               void *out, int out_dtype, int64_t M, int64_t N, int64_t K,
                               void *stream) {
    return matvec_impl(x, x_dtype, packed, scales, out, out_dtype, M, N, K, 0, 0, stream);
}

extern "C" int k3_mxfp4_matvec_cfg(const void *x, int x_dtype, const void *packed,
                                   const void *scales, void *out, int out_dtype, int64_t M,
                                   int64_t N, int64_t K, int rows_per_wave, int groups_per_lane,
                                   void *stream) {
    return matvec_impl(x, x_dtype, packed, scales, out, out_dtype, M, N, K, rows_per_wave,
                       groups_per_lane, stream);
}
