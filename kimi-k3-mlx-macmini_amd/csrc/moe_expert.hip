// One routed expert's SwiGLU / SiTU FFN at batch 1, in two stream-ordered launches.
//
// Reference: LatentMoE.expert_forward (air_llm/models/kimi_k3/moe.py:90-103; k3ref
// k3ref/layers.py:226-234): gate = x Wg^T, up = x Wu^T, act = f(gate, up) in fp32,
// out = act Wd^T -- three projections and two host syncs, weights read once each.
//
// Here:
//   gate/up  every wave owns one (gate row i, up row i) pair, so act[i] = f(g_i, u_i) is
//            produced by the wave that computed both dot products, and written (fp32) to
//            the caller's workspace.  x is staged once per block in LDS; the wave's
//            whole weight stream (both rows, all groups) is issued before the staging.
//   down     the batch-1 MXFP4 GEMV (mxfp4_gemv.hip) with the fp32 act as its activation.
// The launch boundary is the grid-wide dependency between act and the down projection.
// Measured on MI355X, a same-stream kernel boundary costs ~1 us, against ~2.6 us for a
// grid barrier inside one persistent launch plus the re-staging of act after it.
#include <algorithm>
#include <mutex>

#include "moe_common.h"
#include "mxfp4_dot.h"
#include "mxfp4_gemv.h"

namespace k3 {

struct GateUpArgs {
    const void *x;             // [H] bf16 or fp32
    const uint8_t *gp, *gs;    // gate packed [I, H/2], scales [I, H/32]
    const uint8_t *upk, *us;   // up
    float *act;                // [I] fp32 out
    int H, I;
    int act_kind;
    float beta, lbeta;
};

// x tile: XREG 16-byte chunks per thread, every slot written (chunks past the row are
// zeros in slots no lane reads), so no branch can pull an x load behind the weight stream.
template <typename XT>
constexpr int gateup_xreg() { return sizeof(XT) == 2 ? 4 : 8; }

template <typename XT, int GA>
__global__ __launch_bounds__(256) void expert_gateup_kernel(GateUpArgs a) {
    extern __shared__ uint4 smem[];
    constexpr int CPG = XTile<XT>::kChunks;
    constexpr int XREG = gateup_xreg<XT>();
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int GH = a.H >> 5;
    const uint32_t rowA = static_cast<uint32_t>(a.H >> 1);
    const int xchunks = GH * CPG;

    // 1. activation chunks first (small, L2-resident after the first blocks)
    uint4 xr[XREG];
    {
        const auto rx = make_rsrc(a.x, static_cast<uint32_t>(xchunks * 16));
#pragma unroll
        for (int k = 0; k < XREG; ++k) {
            const int c = threadIdx.x + 256 * k;
            xr[k] = buf_load16(rx, c < xchunks ? static_cast<uint32_t>(c) * 16u : kOobOffset);
        }
    }

    // 2. the gate and up rows of pair i, and their scale bytes
    const int i = blockIdx.x * 4 + wave;
    const bool has = i < a.I;
    const auto rg = make_rsrc(a.gp, static_cast<uint32_t>(a.I) * rowA);
    const auto ru = make_rsrc(a.upk, static_cast<uint32_t>(a.I) * rowA);
    const auto rgs = make_rsrc(a.gs, static_cast<uint32_t>(a.I * GH));
    const auto rus = make_rsrc(a.us, static_cast<uint32_t>(a.I * GH));
    uint4 wg[GA], wu[GA];
    uint32_t sg[GA], su[GA];
#pragma unroll
    for (int u = 0; u < GA; ++u) {
        const int g = u * 64 + lane;
        const bool ok = has && g < GH;
        const uint32_t off = ok ? static_cast<uint32_t>(i) * rowA + g * 16u : kOobOffset;
        const uint32_t soff = ok ? static_cast<uint32_t>(i * GH + g) : kOobOffset;
        wg[u] = buf_load16_nt(rg, off);
        wu[u] = buf_load16_nt(ru, off);
        sg[u] = __builtin_amdgcn_raw_buffer_load_b8(rgs, soff, 0, 2);
        su[u] = __builtin_amdgcn_raw_buffer_load_b8(rus, soff, 0, 2);
    }

    // 3. stage x (swizzled chunk order, every slot written)
#pragma unroll
    for (int k = 0; k < XREG; ++k) {
        const int c = threadIdx.x + 256 * k;
        smem[XTile<XT>::slot(c / CPG, c % CPG)] = xr[k];
    }
    __syncthreads();

    // 4. both dot products, group by group in issue order
    float accg = 0.f, accu = 0.f;
#pragma unroll
    for (int u = 0; u < GA; ++u) {
        const int g = u * 64 + lane;
        if (g < GH) {
            XChunk<XT> xc[CPG];
#pragma unroll
            for (int q = 0; q < CPG; ++q) xc[q] = reinterpret_cast<const XChunk<XT> *>(smem)[XTile<XT>::slot(g, q)];
            accg = fmaf(group_dot(wg[u], xc), e8m0_to_f32(sg[u]), accg);
            accu = fmaf(group_dot(wu[u], xc), e8m0_to_f32(su[u]), accu);
        }
    }
    accg = wave_sum_to_lane63(accg);
    accu = wave_sum_to_lane63(accu);
    if (lane == 63 && has) a.act[i] = act_fn(accg, accu, a.act_kind, a.beta, a.lbeta);
}

template <typename XT, int GA>
static int launch_gateup(const GateUpArgs &a, hipStream_t st) {
    const size_t lds = static_cast<size_t>(256) * gateup_xreg<XT>() * 16;
    expert_gateup_kernel<XT, GA><<<dim3(static_cast<unsigned>(cdiv(a.I, 4))), 256, lds, st>>>(a);
    return check_hip(hipGetLastError(), "expert ffn: gate/up launch");
}

template <typename XT>
static int dispatch_gateup(const GateUpArgs &a, hipStream_t st) {
    const int GH = a.H / 32;
    if (GH <= 64) return launch_gateup<XT, 1>(a, st);
    if (GH <= 128) return launch_gateup<XT, 2>(a, st);
    if (GH <= 256) return launch_gateup<XT, 4>(a, st);
    return set_error(K3_ERR_SHAPE, "expert ffn: H=%d exceeds 8192", a.H);
}

// Scratch of the allocation-free entry point: act for I <= kNoAllocMaxI.  One copy per GPU,
// held until the process ends; host code addresses it only through the pointer that
// hipGetSymbolAddress returns for the current device (the array's name is a host-side
// stand-in, not a device address).
constexpr int64_t kNoAllocMaxI = 16384;
static __device__ __align__(256) float scratch[kNoAllocMaxI];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device, resolved once per device.
static int scratch_ptr(void **ptr) {
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "no-alloc expert ffn: current device");
    if (rc) return rc;
    if (dev < 0 || dev >= kMaxDevices) return set_error(K3_ERR_HIP, "no-alloc expert ffn: device %d", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "no-alloc expert ffn: scratch address");
        if (rc) return rc;
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return K3_OK;
}

}  // namespace k3

using namespace k3;

extern "C" int64_t k3_expert_ffn_workspace_size(int64_t I) { return ((I * 4 + 255) / 256) * 256; }

extern "C" int k3_expert_ffn(const void *x, int x_dtype, const void *gate_packed, const void *gate_scales,
                             const void *up_packed, const void *up_scales, const void *down_packed,
                             const void *down_scales, void *out, int out_dtype, int64_t H, int64_t I,
                             int act_kind, float beta, float linear_beta, void *workspace,
                             int64_t workspace_bytes, void *stream);

extern "C" int k3_expert_ffn_noalloc(const void *x, int x_dtype, const void *gate_packed, const void *gate_scales,
                                     const void *up_packed, const void *up_scales, const void *down_packed,
                                     const void *down_scales, void *out, int out_dtype, int64_t H, int64_t I,
                                     int act_kind, float beta, float linear_beta, void *stream) {
    if (I > kNoAllocMaxI)
        return set_error(K3_ERR_WORKSPACE, "no-alloc expert ffn: I=%lld exceeds the %lld values of its scratch",
                         (long long)I, (long long)kNoAllocMaxI);
    void *ws = nullptr;
    const int rc = scratch_ptr(&ws);
    if (rc) return rc;
    return k3_expert_ffn(x, x_dtype, gate_packed, gate_scales, up_packed, up_scales, down_packed, down_scales, out,
                         out_dtype, H, I, act_kind, beta, linear_beta, ws,
                         static_cast<int64_t>(sizeof(float)) * kNoAllocMaxI, stream);
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
    if (H <= 0 || I <= 0 || H % 128 || I % 128 || H > 8192)
        return set_error(K3_ERR_SHAPE, "expert ffn: H=%lld and I=%lld must be positive multiples of 128, H <= 8192",
                         (long long)H, (long long)I);
    if (workspace_bytes < k3_expert_ffn_workspace_size(I))
        return set_error(K3_ERR_WORKSPACE, "expert ffn: workspace %lld < %lld bytes", (long long)workspace_bytes,
                         (long long)k3_expert_ffn_workspace_size(I));
    if (!aligned16(x) || !aligned16(gate_packed) || !aligned16(up_packed) || !aligned16(down_packed) ||
        !aligned16(workspace))
        return set_error(K3_ERR_ALIGN, "expert ffn: x, packed weights and workspace must be 16-byte aligned");
    if (H * I / 2 >= (1ll << 31)) return set_error(K3_ERR_SHAPE, "expert ffn: projection too large");
    if (gemv_token_tile(I, 0) == 0) return set_error(K3_ERR_SHAPE, "expert ffn: I=%lld too large", (long long)I);
    auto st = static_cast<hipStream_t>(stream);
    GateUpArgs a{};
    a.x = x;
    a.gp = static_cast<const uint8_t *>(gate_packed);
    a.gs = static_cast<const uint8_t *>(gate_scales);
    a.upk = static_cast<const uint8_t *>(up_packed);
    a.us = static_cast<const uint8_t *>(up_scales);
    a.act = static_cast<float *>(workspace);
    a.H = static_cast<int>(H);
    a.I = static_cast<int>(I);
    a.act_kind = act_kind;
    a.beta = beta;
    a.lbeta = linear_beta;
    int rc = x_dtype == K3_BF16 ? dispatch_gateup<uint16_t>(a, st) : dispatch_gateup<float>(a, st);
    if (rc) return rc;
    GemvArgs d{};
    d.x = a.act;
    d.ldx = I;
    d.packed = down_packed;
    d.scales = down_scales;
    d.out = out;
    d.ldo = H;
    d.M = 1;
    d.N = H;
    d.K = I;
    d.x_bf16 = 0;
    d.out_bf16 = out_dtype == K3_BF16;
    int rpw, gpl;
    gemv_default_cfg(H, I, &rpw, &gpl);
    return gemv_launch(d, rpw, gpl, st);
}
