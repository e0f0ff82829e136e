// Kimi Delta Attention recurrent step for one token: the state update and read-out of
// every value head, in place on the fp32 state.
//
// Reference: KDAAttention._recurrent (air_llm/models/kimi_k3/attention_kda.py:65-90), the
// upstream naive_recurrent_kda (k3ref/_vendor/kda_naive.py:46-60):
//   S = S * exp(g)[:, None];  S = S + (beta k) (x) (v - k . S);  o = (scale q) . S
// with S [K, V] per value head, g the per-key-channel log decay.
//
// The state is the whole cost: 96 heads x 128 x 128 fp32 = 6 MiB read and written per
// token.  A block owns 32 value columns of one head, so every column's reduction over the
// 128 key channels stays inside the block and the state is read and written exactly once:
// thread t holds rows r, r + 32, r + 64, r + 96 (r = t / 8) of columns 4 (t % 8) .. +3, so
// eight lanes read one 128-byte row segment.  The two reductions over the key channels
// (k . S' for the delta, q . S'' for the read-out) run as xor shuffles inside a wave, then
// across the four waves through LDS in a fixed order.
#include "k3_common.h"

namespace k3 {
namespace {

constexpr int kKdaK = 128;   // key channels (state rows) per head
constexpr int kKdaVS = 32;   // value columns per block

struct KdaArgs {
    const void *q, *k;        // [HQ, K]
    const void *v;            // [HV, V]
    const void *g;            // [HV, K] log decay
    const void *beta;         // [HV]
    int in_bf16;              // q, k, v, g, beta: bf16 (1) or fp32 (0)
    float *S;                 // [HV, K, V] fp32, updated in place
    void *out;                // [HV, V]
    int out_bf16;
    int HV, G, V;             // G = HV / HQ value heads per q/k head
    float scale;
};

__device__ __forceinline__ float ldx(const void *p, int64_t i, int bf) {
    return bf ? bf16_to_f32(static_cast<const uint16_t *>(p)[i]) : static_cast<const float *>(p)[i];
}

// sum over the 8 lanes of a wave that share lane % 8 (the wave's 8 row groups)
__device__ __forceinline__ float sum_row_groups(float x) {
    x += __shfl_xor(x, 8);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
}

__global__ __launch_bounds__(256) void kda_decode_kernel(KdaArgs a) {
    __shared__ float red[2][4][kKdaVS];
    const int nvb = a.V / kKdaVS;
    const int h = blockIdx.x / nvb, vb = blockIdx.x % nvb;
    const int hq = h / a.G;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int cg = t & 7, r = t >> 3;
    const int c0 = vb * kKdaVS + 4 * cg;
    const int bf = a.in_bf16;
    // 1. the four state rows of this thread, then the per-row and per-column scalars
    float *Sp[4];
    float4 x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        Sp[j] = a.S + (static_cast<int64_t>(h) * kKdaK + r + 32 * j) * a.V + c0;
        x[j] = *reinterpret_cast<const float4 *>(Sp[j]);
    }
    float kk[4], qq[4], dk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        kk[j] = ldx(a.k, static_cast<int64_t>(hq) * kKdaK + r + 32 * j, bf);
        qq[j] = ldx(a.q, static_cast<int64_t>(hq) * kKdaK + r + 32 * j, bf) * a.scale;
        dk[j] = expf(ldx(a.g, static_cast<int64_t>(h) * kKdaK + r + 32 * j, bf));
    }
    const float b = ldx(a.beta, h, bf);
    float vv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) vv[c] = ldx(a.v, static_cast<int64_t>(h) * a.V + c0 + c, bf);
    // 2. decay, then k . S' over the 128 channels
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j].x *= dk[j], x[j].y *= dk[j], x[j].z *= dk[j], x[j].w *= dk[j];
    float p[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        p[0] = fmaf(kk[j], x[j].x, p[0]);
        p[1] = fmaf(kk[j], x[j].y, p[1]);
        p[2] = fmaf(kk[j], x[j].z, p[2]);
        p[3] = fmaf(kk[j], x[j].w, p[3]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) p[c] = sum_row_groups(p[c]);
    if (lane < 8) {
#pragma unroll
        for (int c = 0; c < 4; ++c) red[0][wave][4 * lane + c] = p[c];
    }
    __syncthreads();
    float d[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int i = 4 * cg + c;
        d[c] = vv[c] - (((red[0][0][i] + red[0][1][i]) + red[0][2][i]) + red[0][3][i]);
    }
    // 3. the delta update, written back; then q . S''
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float bk = b * kk[j];
        x[j].x = fmaf(bk, d[0], x[j].x);
        x[j].y = fmaf(bk, d[1], x[j].y);
        x[j].z = fmaf(bk, d[2], x[j].z);
        x[j].w = fmaf(bk, d[3], x[j].w);
        *reinterpret_cast<float4 *>(Sp[j]) = x[j];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) p[c] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        p[0] = fmaf(qq[j], x[j].x, p[0]);
        p[1] = fmaf(qq[j], x[j].y, p[1]);
        p[2] = fmaf(qq[j], x[j].z, p[2]);
        p[3] = fmaf(qq[j], x[j].w, p[3]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) p[c] = sum_row_groups(p[c]);
    if (lane < 8) {
#pragma unroll
        for (int c = 0; c < 4; ++c) red[1][wave][4 * lane + c] = p[c];
    }
    __syncthreads();
    if (t < kKdaVS) {
        const float o = ((red[1][0][t] + red[1][1][t]) + red[1][2][t]) + red[1][3][t];
        const int64_t oi = static_cast<int64_t>(h) * a.V + vb * kKdaVS + t;
        if (a.out_bf16)
            static_cast<uint16_t *>(a.out)[oi] = f32_to_bf16(o);
        else
            static_cast<float *>(a.out)[oi] = o;
    }
}

}  // namespace
}  // namespace k3

using namespace k3;

extern "C" int k3_kda_recurrent_decode(const void *q, const void *k, const void *v, const void *g, const void *beta,
                                       int in_dtype, float *state, void *out, int out_dtype, int64_t qk_heads,
                                       int64_t v_heads, int64_t key_dim, int64_t value_dim, float scale,
                                       void *stream) {
    if (!q || !k || !v || !g || !beta || !state || !out) return set_error(K3_ERR_NULL, "kda decode: null pointer");
    if (in_dtype != K3_F32 && in_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "kda decode: in_dtype %d", in_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "kda decode: out_dtype %d", out_dtype);
    if (key_dim != kKdaK)
        return set_error(K3_ERR_SHAPE, "kda decode: key_dim=%lld; the kernel takes %d", (long long)key_dim, kKdaK);
    if (value_dim <= 0 || value_dim % kKdaVS || value_dim > 4096)
        return set_error(K3_ERR_SHAPE, "kda decode: value_dim=%lld must be a positive multiple of %d, <= 4096",
                         (long long)value_dim, kKdaVS);
    if (qk_heads <= 0 || v_heads <= 0 || v_heads % qk_heads || v_heads > (1 << 20))
        return set_error(K3_ERR_SHAPE, "kda decode: v_heads=%lld must be a positive multiple of qk_heads=%lld",
                         (long long)v_heads, (long long)qk_heads);
    if (!aligned16(state)) return set_error(K3_ERR_ALIGN, "kda decode: the state must be 16-byte aligned");
    KdaArgs a{};
    a.q = q, a.k = k, a.v = v, a.g = g, a.beta = beta;
    a.in_bf16 = in_dtype == K3_BF16;
    a.S = state;
    a.out = out;
    a.out_bf16 = out_dtype == K3_BF16;
    a.HV = static_cast<int>(v_heads);
    a.G = static_cast<int>(v_heads / qk_heads);
    a.V = static_cast<int>(value_dim);
    a.scale = scale;
    const int64_t blocks = v_heads * (value_dim / kKdaVS);
    kda_decode_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, 0, static_cast<hipStream_t>(stream)>>>(a);
    return check_hip(hipGetLastError(), "kda decode launch");
}
