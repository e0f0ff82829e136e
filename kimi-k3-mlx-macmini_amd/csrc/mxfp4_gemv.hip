// Fused MXFP4 matvec / small-M matmul for gfx950 (the batch-1 expert GEMV).
//
// Replaces the reference Metal kernel (air_llm/kernels/metal/mxfp4_matvec.py:29-63), which
// runs one thread per output and walks a packed row byte by byte.  Here:
//
//   * a wave owns RPW weight rows; its 64 lanes sweep the row's 32-element groups, lane l
//     taking groups l, l+64, ... so every 128-bit load of packed nibbles is part of a
//     contiguous 1 KiB wave-wide read (one group = 16 packed bytes = one E8M0 scale);
//   * every lane loads the scale byte of each of its groups (a wave's 64 byte loads are one
//     contiguous 64-byte read), and the activation tokens are staged in LDS once per block,
//     in a swizzled 16-byte-chunk order so the per-lane group reads do not collide on banks;
//   * nibbles become bf16 pairs (bf16 activations: v_cvt_scalef32_pk_bf16_fp4 then
//     v_dot2_f32_bf16) or fp32 pairs (fp32 activations: v_cvt_scalef32_pk_f32_fp4 then
//     fp32 FMA); each group's partial sum is scaled once by its power-of-two E8M0 scale
//     (exact) and accumulated in fp32;
//   * the activation loads are issued first, then the wave's whole weight stream, so the
//     LDS staging waits only for the activations; rows longer than one sweep prefetch the
//     next sweep before consuming the current one; the per-lane partials are summed with a
//     DPP wave reduction.
//
// Numerics: weights are exact (E2M1 x 2^e), products of bf16/fp32 activations with them
// are exact in fp32, accumulation is fp32 -- the same arithmetic class as the reference
// fused kernel, with a different (grouped, then tree) summation order.
#include "k3_common.h"
#include "mxfp4_dot.h"
#include "mxfp4_gemv.h"

#include <type_traits>

namespace k3 {

// Activation tile: XREG 16-byte chunks per thread per token (256 threads), so every thread
// issues a fixed number of x loads and writes every slot of the tile unconditionally.
// Chunks past the row load as zeros and land in slots no lane reads.  (A conditional store
// lets the compiler sink the x load into the branch behind a vmcnt(0), which would make
// the staging wait for the whole weight stream issued after it.)
int xreg_choice(int64_t K, int x_bf16) {
    const int64_t chunks = (K / 32) * (x_bf16 ? 4 : 8);
    if (chunks <= 256 * 4) return 4;
    if (chunks <= 256 * 8) return 8;
    if (chunks <= 256 * 16) return 16;
    return 0;
}

// LOOP == false: one sweep covers the row (G <= 64 * GPL), with no loop or prefetch code, so
// the in-order vmcnt waits of the group loop count exactly the loads issued after each
// group.  LOOP == true: sweeps of 64 * GPL groups, the next sweep's loads issued before the
// current one is consumed (rows longer than one sweep, or forced launch shapes).
template <typename XT, int RPW, int GPL, int MT, int XREG, bool LOOP>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    extern __shared__ uint4 smem[];
    constexpr int CPG = XTile<XT>::kChunks;
    constexpr int TILE = 256 * XREG;  // chunks per token
    const int G = static_cast<int>(a.K >> 5);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t n0 = (static_cast<int64_t>(blockIdx.x) * 4 + wave) * RPW;
    const uint32_t row_bytes = static_cast<uint32_t>(a.K >> 1);
    const int xchunks = G * CPG;

    // 1. activation chunks (small, L2-resident after the first blocks) first
    uint4 xr[MT][XREG];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const auto rx = make_rsrc(static_cast<const XT *>(a.x) + m * a.ldx,
                                  m < a.M ? static_cast<uint32_t>(xchunks * 16) : 0u);
#pragma unroll
        for (int k = 0; k < XREG; ++k) {
            const int c = threadIdx.x + 256 * k;
            xr[m][k] = buf_load16(rx, c < xchunks ? static_cast<uint32_t>(c) * 16u : kOobOffset);
        }
    }

    // 2. the first sweep of this wave's weights and one scale byte per (row, group);
    //    rows past N and groups past G read zeros
    const auto rw = make_rsrc(a.packed, static_cast<uint32_t>(a.N * row_bytes));
    const auto rs = make_rsrc(a.scales, static_cast<uint32_t>(a.N * G));
    uint4 w[RPW][GPL];
    uint32_t sb[RPW][GPL];
    auto load_sweep = [&](int gs) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int64_t n = n0 + r;
#pragma unroll
            for (int u = 0; u < GPL; ++u) {
                const int g = gs + u * kWave + lane;
                const bool ok = n < a.N && g < G;
                w[r][u] = buf_load16_nt(rw, ok ? static_cast<uint32_t>(n) * row_bytes + static_cast<uint32_t>(g) * 16u
                                            : kOobOffset);
                sb[r][u] = __builtin_amdgcn_raw_buffer_load_b8(rs, ok ? static_cast<uint32_t>(n * G + g) : kOobOffset,
                                                               0, 2);
            }
        }
    };
    load_sweep(0);

    // 3. activations to LDS (swizzled chunk order, every slot written)
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int k = 0; k < XREG; ++k) {
            const int c = threadIdx.x + 256 * k;
            smem[m * TILE + XTile<XT>::slot(c / CPG, c % CPG)] = xr[m][k];
        }
    __syncthreads();

    // 4. consume groups in issue order (vmcnt is in order, so group u waits only for its
    //    own loads); each group's partial is scaled once by its power-of-two scale
    float acc[MT][RPW];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[m][r] = 0.f;
    for (int gs = 0;;) {
        uint4 cw[RPW][GPL];
        uint32_t cs[RPW][GPL];
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int u = 0; u < GPL; ++u) cw[r][u] = w[r][u], cs[r][u] = sb[r][u];
        const int next = gs + kWave * GPL;
        if constexpr (LOOP) {
            if (next < G) load_sweep(next);
        }
#pragma unroll
        for (int u = 0; u < GPL; ++u) {
            const int g = gs + u * kWave + lane;
            if (g < G) {
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    if (m < a.M) {
                        XChunk<XT> xc[CPG];
#pragma unroll
                        for (int q = 0; q < CPG; ++q)
                            xc[q] = reinterpret_cast<const XChunk<XT> *>(smem)[m * TILE + XTile<XT>::slot(g, q)];
#pragma unroll
                        for (int r = 0; r < RPW; ++r)
                            acc[m][r] = fmaf(group_dot(cw[r][u], xc), e8m0_to_f32(cs[r][u]), acc[m][r]);
                    }
                }
            }
        }
        if (!LOOP || next >= G) break;
        gs = next;
    }

    // 5. wave reduction and store (lane 63 holds each total)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const float t = wave_sum_to_lane63(acc[m][r]);
            const int64_t n = n0 + r;
            if (lane == 63 && m < a.M && n < a.N) {
                if (a.out_bf16)
                    static_cast<uint16_t *>(a.out)[m * a.ldo + n] = f32_to_bf16(t);
                else
                    static_cast<float *>(a.out)[m * a.ldo + n] = t;
            }
        }
    }
}

template <typename XT, int RPW, int GPL, int MT, int XREG>
static int launch_one(const GemvArgs &a, hipStream_t st) {
    const bool loop = (a.K >> 5) > kWave * GPL;
    const size_t lds = static_cast<size_t>(MT) * 256 * XREG * 16;
    if (lds > kGemvMaxLds)
        return set_error(K3_ERR_SHAPE, "mxfp4 matvec: K=%lld needs %zu bytes of LDS (max %zu)", (long long)a.K, lds,
                         kGemvMaxLds);
    auto kern = loop ? &gemv_kernel<XT, RPW, GPL, MT, XREG, true> : &gemv_kernel<XT, RPW, GPL, MT, XREG, false>;
    if (lds > 64 * 1024) {  // above the default dynamic-LDS limit: opt in (gfx950 has 160 KiB)
        int rc = check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)),
                           "mxfp4 matvec: raise LDS limit");
        if (rc) return rc;
    }
    const dim3 grid(static_cast<unsigned>(cdiv(a.N, 4 * RPW)));
    kern<<<grid, 256, lds, st>>>(a);
    return check_hip(hipGetLastError(), "mxfp4 matvec launch");
}

template <typename XT, int MT, int XREG>
static int dispatch_cfg(const GemvArgs &a, int rpw, int gpl, hipStream_t st) {
#define K3_CFG(R, U) \
    if (rpw == R && gpl == U) return launch_one<XT, R, U, MT, XREG>(a, st);
    K3_CFG(1, 4) K3_CFG(2, 4) K3_CFG(1, 2) K3_CFG(2, 2) K3_CFG(4, 2) K3_CFG(1, 1) K3_CFG(2, 1) K3_CFG(4, 1)
    if constexpr (MT == 1) { K3_CFG(8, 1) }
#undef K3_CFG
    return set_error(K3_ERR_SHAPE, "mxfp4 matvec: no kernel for rpw=%d gpl=%d", rpw, gpl);
}

// Default launch shape: cover K in at most one or two sweeps and keep >= ~2 blocks per CU.
// Rows of up to 2048 values (one sweep of one group per lane) take two rows per wave from
// 1024 rows on: the expert's down projection ([7168 x 2048], 896 blocks) measured 9.53 ->
// 9.39 us per expert step against four rows per wave (448 blocks), 9.60 us with one.
void gemv_default_cfg(int64_t N, int64_t K, int *rpw, int *gpl) {
    const int64_t G = K / 32;
    *gpl = G > 128 ? 4 : (G > 64 ? 2 : 1);
    if (*gpl == 1)
        *rpw = N >= 4 * 256 ? 2 : 1;
    else if (*gpl == 2)
        *rpw = N >= 8 * 512 ? 4 : (N >= 4 * 512 ? 2 : 1);
    else
        *rpw = N >= 4 * 2 * 512 ? 2 : 1;
    if (*rpw == 8 && *gpl != 1) *rpw = 4;
    if (*rpw == 4 && *gpl == 4) *rpw = 2;
}

// Tokens per launch: up to 4 share one weight pass while their activation tiles fit the LDS
// (8 chunks per thread per token), otherwise one.
int gemv_token_tile(int64_t K, int x_bf16) {
    const int xr = xreg_choice(K, x_bf16);
    return xr == 0 ? 0 : (xr <= 8 ? 4 : 1);
}

template <typename XT>
static int dispatch_x(const GemvArgs &a, int rpw, int gpl, hipStream_t st) {
    const int xr = xreg_choice(a.K, std::is_same<XT, uint16_t>::value);
    if (a.M == 1) {
        if (xr == 4) return dispatch_cfg<XT, 1, 4>(a, rpw, gpl, st);
        if (xr == 8) return dispatch_cfg<XT, 1, 8>(a, rpw, gpl, st);
        if (xr == 16) return dispatch_cfg<XT, 1, 16>(a, rpw, gpl, st);
    } else {
        if (xr == 4) return dispatch_cfg<XT, 4, 4>(a, rpw, gpl, st);
        if (xr == 8) return dispatch_cfg<XT, 4, 8>(a, rpw, gpl, st);
    }
    return set_error(K3_ERR_SHAPE, "mxfp4 matvec: K=%lld is too long for %d token(s) per launch", (long long)a.K,
                     a.M);
}

int gemv_launch(const GemvArgs &a, int rpw, int gpl, hipStream_t st) {
    return a.x_bf16 ? dispatch_x<uint16_t>(a, rpw, gpl, st) : dispatch_x<float>(a, rpw, gpl, st);
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
                       int out_dtype, int64_t M, int64_t N, int64_t K, void *stream) {
    int rc = gemv_validate(x, x_dtype, packed, scales, out, out_dtype, M, N, K);
    if (rc) return rc;
    if (M == 0 || N == 0) return K3_OK;
    int rpw, gpl;
    gemv_default_cfg(N, K, &rpw, &gpl);
    if (M > 1 && rpw == 8) rpw = 4;
    const size_t xsz = x_dtype == K3_BF16 ? 2 : 4;
    const size_t osz = out_dtype == K3_BF16 ? 2 : 4;
    const int mt = gemv_token_tile(K, x_dtype == K3_BF16);
    if (mt == 0)
        return set_error(K3_ERR_SHAPE, "mxfp4 matvec: K=%lld exceeds the %d-element activation tile", (long long)K,
                         x_dtype == K3_BF16 ? 32768 : 16384);
    auto st = static_cast<hipStream_t>(stream);
    for (int64_t m0 = 0; m0 < M; m0 += mt) {  // token tiles share one weight pass
        GemvArgs a{};
        a.x = static_cast<const char *>(x) + m0 * K * xsz;
        a.ldx = K;
        a.packed = packed;
        a.scales = scales;
        a.out = static_cast<char *>(out) + m0 * N * osz;
        a.ldo = N;
        a.M = static_cast<int>(std::min<int64_t>(mt, M - m0));
        a.N = N;
        a.K = K;
        a.x_bf16 = x_dtype == K3_BF16;
        a.out_bf16 = out_dtype == K3_BF16;
        rc = gemv_launch(a, rpw, gpl, st);
        if (rc) return rc;
    }
    return K3_OK;
}

extern "C" int k3_mxfp4_matvec(const void *x, int x_dtype, const void *packed, const void *scales,
                               void *out, int out_dtype, int64_t M, int64_t N, int64_t K,
                               void *stream) {
    return matvec_impl(x, x_dtype, packed, scales, out, out_dtype, M, N, K, stream);
}
