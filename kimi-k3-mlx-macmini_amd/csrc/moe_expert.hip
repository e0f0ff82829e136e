// One routed expert's SwiGLU / SiTU FFN at batch 1, in a single persistent launch.
//
// Reference: LatentMoE.expert_forward (air_llm/models/kimi_k3/moe.py:90-103; k3ref
// k3ref/layers.py:226-234): gate = x Wg^T, up = x Wu^T, act = f(gate, up) in fp32,
// out = act Wd^T -- three projections and two host syncs, weights read once each.
//
// Here the whole expert is one kernel of 4-wave blocks:
//   phase A  every wave owns one (gate row i, up row i) pair, so act[i] = f(g_i, u_i) is
//            produced by the wave that computed both dot products;
//   prefetch waves 1-3 load their down-projection rows (RB per wave) and scales into
//            registers at kernel start, so that stream overlaps phase A and the barrier;
//   barrier  wave 0 (no loads in flight) copies the block's act values to the workspace
//            with coherent stores and publishes the block's epoch flag (moe_common.h);
//   phase B  act is staged in LDS and waves 1-3 reduce their prefetched rows.
// Tails and idle rows read through buffer loads that return zeros out of range.
#include <algorithm>

#include "moe_common.h"
#include "mxfp4_dot.h"

namespace k3 {

struct FfnArgs {
    const void *x;           // [H] bf16 or fp32
    const uint8_t *gp, *gs;  // gate packed [I, H/2], scales [I, H/32]
    const uint8_t *upk, *us; // up
    const uint8_t *dp, *ds;  // down packed [H, I/2], scales [H, I/32]
    uint32_t *ws;            // workspace: barrier region, then act [I] fp32
    float *act;
    void *out;               // [H] fp32 or bf16
    int H, I;
    int out_bf16;
    int act_kind;
    float beta, lbeta;
};

template <typename XT, int GA, int RB, int GB>
__global__ __launch_bounds__(256) void expert_ffn_kernel(FfnArgs a) {
    extern __shared__ uint4 smem[];
    __shared__ uint32_t epoch_s;
    __shared__ float act_s[4];
    constexpr int CPGX = XTile<XT>::kChunks;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int GH = a.H >> 5, GI = a.I >> 5;
    const uint32_t rowA = static_cast<uint32_t>(a.H >> 1), rowB = static_cast<uint32_t>(a.I >> 1);
    uint4 *xs = smem;
    uint4 *as = smem + GH * CPGX;
    barrier_epoch(a.ws, &epoch_s);

    // ---- activations first (small, L2-resident after the first blocks), so the LDS
    //      staging below waits only for them and not for the weight stream
    constexpr int XREG = 8;
    const int xchunks = GH * CPGX;
    uint4 xreg[XREG];
    {
        const auto xr = make_rsrc(a.x, static_cast<uint32_t>(xchunks * 16));
#pragma unroll
        for (int k = 0; k < XREG; ++k) {
            const int c = threadIdx.x + 256 * k;
            xreg[k] = buf_load16(xr, c < xchunks ? static_cast<uint32_t>(c) * 16u : kOobOffset);
        }
    }

    // ---- phase A operands: gate/up row pair i
    const int i = blockIdx.x * 4 + wave;
    const bool has_a = i < a.I;
    const auto rg = make_rsrc(a.gp, static_cast<uint32_t>(a.I) * rowA);
    const auto ru = make_rsrc(a.upk, static_cast<uint32_t>(a.I) * rowA);
    const auto rgs = make_rsrc(a.gs, static_cast<uint32_t>(a.I * GH));
    const auto rus = make_rsrc(a.us, static_cast<uint32_t>(a.I * GH));
    uint4 wg_[GA], wu_[GA];
    uint32_t sg_[GA], su_[GA];
#pragma unroll
    for (int u = 0; u < GA; ++u) {
        const int g = u * 64 + lane;
        const bool v = has_a && g < GH;
        const uint32_t off = v ? static_cast<uint32_t>(i) * rowA + g * 16u : kOobOffset;
        const uint32_t soff = v ? scale_dword_off(static_cast<uint32_t>(i * GH), g) : kOobOffset;
        wg_[u] = buf_load16(rg, off);
        wu_[u] = buf_load16(ru, off);
        sg_[u] = buf_load4(rgs, soff);
        su_[u] = buf_load4(rus, soff);
    }

    // ---- phase B operands, prefetched by waves 1-3: rows n = pw + rb * PW
    const int PW = gridDim.x * 3;
    const int pw = blockIdx.x * 3 + wave - 1;
    const auto rd = make_rsrc(a.dp, static_cast<uint32_t>(a.H) * rowB);
    const auto rds = make_rsrc(a.ds, static_cast<uint32_t>(a.H * GI));
    uint4 wd_[RB][GB];
    uint32_t sd_[RB][GB];
    if (wave > 0) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int n = pw + rb * PW;
#pragma unroll
            for (int u = 0; u < GB; ++u) {
                const int g = u * 64 + lane;
                const bool v = n < a.H && g < GI;
                wd_[rb][u] = buf_load16(rd, v ? static_cast<uint32_t>(n) * rowB + g * 16u : kOobOffset);
                sd_[rb][u] = buf_load4(rds, v ? scale_dword_off(static_cast<uint32_t>(n * GI), g) : kOobOffset);
            }
        }
    }

    // ---- stage x, then phase A
#pragma unroll
    for (int k = 0; k < XREG; ++k) {
        const int c = threadIdx.x + 256 * k;
        if (c < xchunks) xs[XTile<XT>::slot(c / CPGX, c % CPGX)] = xreg[k];
    }
    __syncthreads();
    float accg = 0.f, accu = 0.f;
#pragma unroll
    for (int u = 0; u < GA; ++u) {
        const int g = u * 64 + lane;
        if (has_a && g < GH) {
            XChunk<XT> xc[CPGX];
#pragma unroll
            for (int q = 0; q < CPGX; ++q) xc[q] = reinterpret_cast<const XChunk<XT> *>(xs)[XTile<XT>::slot(g, q)];
            const uint32_t so = static_cast<uint32_t>(i * GH);
            accg = fmaf(group_dot(wg_[u], xc), e8m0_to_f32(scale_byte(sg_[u], so, g)), accg);
            accu = fmaf(group_dot(wu_[u], xc), e8m0_to_f32(scale_byte(su_[u], so, g)), accu);
        }
    }
    accg = wave_sum_to_lane63(accg);
    accu = wave_sum_to_lane63(accu);
    if (lane == 63) act_s[wave] = act_fn(accg, accu, a.act_kind, a.beta, a.lbeta);
    __syncthreads();

    // ---- publish act, grid barrier (wave 0)
    if (wave == 0) {
        if (lane < 4 && blockIdx.x * 4 + lane < a.I) store_coherent(a.act + blockIdx.x * 4 + lane, act_s[lane]);
        barrier_publish_and_wait(a.ws, epoch_s + 1);
    }
    __syncthreads();
    barrier_advance_epoch(a.ws, epoch_s, 1);

    // ---- stage act (coherent loads), phase B on waves 1-3
    {
        const auto ra = make_rsrc(a.act, static_cast<uint32_t>(a.I) * 4u);
        for (int c = threadIdx.x; c < GI * 8; c += 256) as[XTile<float>::slot(c >> 3, c & 7)] = load16_coherent(ra, c * 16u);
    }
    __syncthreads();
    if (wave == 0) return;
    float acc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = 0.f;
#pragma unroll
    for (int u = 0; u < GB; ++u) {
        const int g = u * 64 + lane;
        if (g < GI) {
            float4 ac[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) ac[q] = reinterpret_cast<const float4 *>(as)[XTile<float>::slot(g, q)];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const int n = pw + rb * PW;
                acc[rb] = fmaf(group_dot(wd_[rb][u], ac),
                               e8m0_to_f32(scale_byte(sd_[rb][u], static_cast<uint32_t>(n * GI), g)), acc[rb]);
            }
        }
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int n = pw + rb * PW;
        const float t = wave_sum_to_lane63(acc[rb]);
        if (lane == 63 && n < a.H) {
            if (a.out_bf16)
                static_cast<uint16_t *>(a.out)[n] = f32_to_bf16(t);
            else
                static_cast<float *>(a.out)[n] = t;
        }
    }
}

int resident_blocks(const void *kernel, int block_threads, size_t lds_bytes, int *out) {
    int dev = 0, cus = 0, per_cu = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    rc = check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
    if (rc) return rc;
    rc = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block_threads, lds_bytes),
                   "occupancy query");
    if (rc) return rc;
    *out = cus * per_cu;
    return K3_OK;
}

template <typename XT, int GA, int RB, int GB>
static int launch_ffn(const FfnArgs &a, hipStream_t st) {
    const int GH = a.H / 32, GI = a.I / 32;
    const size_t lds = static_cast<size_t>(GH) * XTile<XT>::kChunks * 16 + static_cast<size_t>(GI) * 128;
    auto kern = &expert_ffn_kernel<XT, GA, RB, GB>;
    int cap = 0;
    int rc = resident_blocks(reinterpret_cast<const void *>(kern), 256, lds, &cap);
    if (rc) return rc;
    const int blocks = static_cast<int>(std::max<int64_t>(cdiv(a.I, 4), cdiv(a.H, 3 * RB)));
    if (blocks > cap || blocks > kMaxGridBlocks)
        return set_error(K3_ERR_SHAPE, "expert ffn: %d blocks exceed the %d resident blocks", blocks, cap);
    kern<<<dim3(blocks), 256, lds, st>>>(a);
    return check_hip(hipGetLastError(), "expert ffn launch");
}

template <typename XT>
static int dispatch_ffn(const FfnArgs &a, hipStream_t st) {
    const int GH = a.H / 32, GI = a.I / 32;
    const int ga = GH <= 128 ? 2 : (GH <= 256 ? 4 : 0);
    if (GH * XTile<XT>::kChunks > 256 * 8)
        return set_error(K3_ERR_SHAPE, "expert ffn: H=%d too wide for the fused kernel", a.H);
    const int gb = GI <= 64 ? 1 : (GI <= 128 ? 2 : 0);
    if (!ga || !gb) return set_error(K3_ERR_SHAPE, "expert ffn: H=%d I=%d outside the fused kernel", a.H, a.I);
    // down rows per prefetching wave: 3 * (I / 4) waves must cover H rows
    const int64_t need = cdiv(a.H, 3 * cdiv(a.I, 4));
    const int rb = need <= 2 ? 2 : (need <= 4 ? 4 : (need <= 6 ? 6 : 8));
#define K3_FFN(GA_, RB_, GB_) \
    if (ga == GA_ && rb == RB_ && gb == GB_) return launch_ffn<XT, GA_, RB_, GB_>(a, st);
    K3_FFN(2, 2, 1) K3_FFN(2, 2, 2) K3_FFN(2, 4, 1) K3_FFN(2, 4, 2) K3_FFN(2, 6, 1) K3_FFN(2, 8, 1)
    K3_FFN(4, 2, 1) K3_FFN(4, 2, 2) K3_FFN(4, 4, 1) K3_FFN(4, 4, 2) K3_FFN(4, 6, 1) K3_FFN(4, 8, 1)
#undef K3_FFN
    return set_error(K3_ERR_SHAPE, "expert ffn: no kernel");
}

}  // namespace k3

using namespace k3;

extern "C" int64_t k3_expert_ffn_workspace_size(int64_t I) {
    return static_cast<int64_t>(kBarrierRegion) + ((I * 4 + 255) / 256) * 256;
}

extern "C" int k3_expert_ffn(const void *x, int x_dtype, const void *gate_packed, const void *gate_scales,
                             const void *up_packed, const void *up_scales, const void *down_packed,
                             const void *down_scales, void *out, int out_dtype, int64_t H, int64_t I,
                             int act_kind, float beta, float linear_beta, void *workspace,
                             int64_t workspace_bytes, void *stream) {
    if (!x || !gate_packed || !gate_scales || !up_packed || !up_scales || !down_packed || !down_scales ||
        !out || !workspace)
        return set_error(K3_ERR_NULL, "expert ffn: null pointer");
    if (x_dtype != K3_F32 && x_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "expert ffn: x_dtype");
    if (out_dtype != K3_F32 && out_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "expert ffn: out_dtype");
    if (act_kind != K3_ACT_SILU && act_kind != K3_ACT_SITU) return set_error(K3_ERR_SHAPE, "expert ffn: act_kind");
    if (H <= 0 || I <= 0 || H % 128 || I % 128)
        return set_error(K3_ERR_SHAPE, "expert ffn: H=%lld and I=%lld must be positive multiples of 128",
                         (long long)H, (long long)I);
    if (workspace_bytes < k3_expert_ffn_workspace_size(I))
        return set_error(K3_ERR_WORKSPACE, "expert ffn: workspace %lld < %lld bytes", (long long)workspace_bytes,
                         (long long)k3_expert_ffn_workspace_size(I));
    if (!aligned16(x) || !aligned16(gate_packed) || !aligned16(up_packed) || !aligned16(down_packed) ||
        !aligned16(workspace))
        return set_error(K3_ERR_ALIGN, "expert ffn: x, packed weights and workspace must be 16-byte aligned");
    if (H * I / 2 >= (1ll << 31)) return set_error(K3_ERR_SHAPE, "expert ffn: projection too large");
    FfnArgs a{};
    a.x = x;
    a.gp = static_cast<const uint8_t *>(gate_packed);
    a.gs = static_cast<const uint8_t *>(gate_scales);
    a.upk = static_cast<const uint8_t *>(up_packed);
    a.us = static_cast<const uint8_t *>(up_scales);
    a.dp = static_cast<const uint8_t *>(down_packed);
    a.ds = static_cast<const uint8_t *>(down_scales);
    a.ws = static_cast<uint32_t *>(workspace);
    a.act = reinterpret_cast<float *>(static_cast<char *>(workspace) + kBarrierRegion);
    a.out = out;
    a.H = static_cast<int>(H);
    a.I = static_cast<int>(I);
    a.out_bf16 = out_dtype == K3_BF16;
    a.act_kind = act_kind;
    a.beta = beta;
    a.lbeta = linear_beta;
    auto st = static_cast<hipStream_t>(stream);
    return x_dtype == K3_BF16 ? dispatch_ffn<uint16_t>(a, st) : dispatch_ffn<float>(a, st);
}
