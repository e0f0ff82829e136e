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
#include "dense_rows.h"

namespace k3 {
namespace {

constexpr int kKdaK = 128;   // key channels (state rows) per head
constexpr int kKdaVS = 32;   // value columns per block

struct KdaArgs {
    const void *q, *k;        // [T, HQ, K]
    const void *v;            // [T, HV, V]
    const void *g;            // [T, HV, K] log decay
    const void *beta;         // [T, HV]
    int in_bf16;              // q, k, v, g, beta: bf16 (1) or fp32 (0)
    float *S;                 // [HV, K, V] fp32, updated in place
    void *out;                // [T, HV, V]
    int out_bf16;
    int HV, G, V, T;          // G = HV / HQ value heads per q/k head
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

// The update of one block's 32 columns of head h's state, given this thread's four rows'
// key values kk, scaled query values qq and decay factors dk, its four columns' values vv
// and the head's beta.  x holds the thread's state values (loaded by the caller, stored by
// the caller once its tokens are done).
// Returns the read-out of column t (valid in threads t < 32).
__device__ __forceinline__ float kda_apply(float4 (&x)[4], const float (&kk)[4],
                                           const float (&qq)[4], const float (&dk)[4], const float (&vv)[4], float b,
                                           float (*red)[4][kKdaVS]) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, cg = t & 7;
    // decay, then k . S' over the 128 channels
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
    // the delta update, written back; then q . S''
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float bk = b * kk[j];
        x[j].x = fmaf(bk, d[0], x[j].x);
        x[j].y = fmaf(bk, d[1], x[j].y);
        x[j].z = fmaf(bk, d[2], x[j].z);
        x[j].w = fmaf(bk, d[3], x[j].w);
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
    return t < kKdaVS ? ((red[1][0][t] + red[1][1][t]) + red[1][2][t]) + red[1][3][t] : 0.f;
}

__device__ __forceinline__ void kda_store_state(const float4 (&x)[4], float *const (&Sp)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<float4 *>(Sp[j]) = x[j];
}

// the four state rows t/8 + 32j of columns c0 .. c0+3 of head h
__device__ __forceinline__ void kda_load_state(float *S, int h, int V, int c0, float4 (&x)[4], float *(&Sp)[4]) {
    const int r = threadIdx.x >> 3;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        Sp[j] = S + (static_cast<int64_t>(h) * kKdaK + r + 32 * j) * V + c0;
        x[j] = *reinterpret_cast<const float4 *>(Sp[j]);
    }
}

// T tokens in order; the block's state columns stay in registers between them, so the
// state is read and written once whatever T is.  The next token's inputs are loaded while
// the current one is reduced.
template <bool MULTI>
__global__ __launch_bounds__(256) void kda_decode_kernel(KdaArgs a) {
    __shared__ float red[2][4][kKdaVS];
    const int nvb = a.V / kKdaVS;
    const int h = blockIdx.x / nvb, vb = blockIdx.x % nvb;
    const int hq = h / a.G, HQ = a.HV / a.G;
    const int t = threadIdx.x, cg = t & 7, r = t >> 3;
    const int c0 = vb * kKdaVS + 4 * cg;
    const int bf = a.in_bf16;
    float *Sp[4];
    float4 x[4];
    kda_load_state(a.S, h, a.V, c0, x, Sp);
    float kk[4], qq[4], dk[4], vv[4], b;
    auto load = [&](int i, float(&k_)[4], float(&q_)[4], float(&d_)[4], float(&v_)[4], float &b_) {
        const int64_t qo = (static_cast<int64_t>(i) * HQ + hq) * kKdaK, go = (static_cast<int64_t>(i) * a.HV + h) * kKdaK;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            k_[j] = ldx(a.k, qo + r + 32 * j, bf);
            q_[j] = ldx(a.q, qo + r + 32 * j, bf) * a.scale;
            d_[j] = ldx(a.g, go + r + 32 * j, bf);
        }
        const int64_t vo = (static_cast<int64_t>(i) * a.HV + h) * a.V + c0;
#pragma unroll
        for (int c = 0; c < 4; ++c) v_[c] = ldx(a.v, vo + c, bf);
        b_ = ldx(a.beta, static_cast<int64_t>(i) * a.HV + h, bf);
    };
    load(0, kk, qq, dk, vv, b);
    const int T = MULTI ? a.T : 1;
    for (int i = 0; i < T; ++i) {
        float nk[4], nq[4], nd[4], nv[4], nb = 0.f;
        if (MULTI && i + 1 < T) load(i + 1, nk, nq, nd, nv, nb);
#pragma unroll
        for (int j = 0; j < 4; ++j) dk[j] = expf(dk[j]);
        const float o = kda_apply(x, kk, qq, dk, vv, b, red);
        if (t < kKdaVS) {
            const int64_t oi = (static_cast<int64_t>(i) * a.HV + h) * a.V + vb * kKdaVS + t;
            if (a.out_bf16)
                static_cast<uint16_t *>(a.out)[oi] = f32_to_bf16(o);
            else
                static_cast<float *>(a.out)[oi] = o;
        }
        if (MULTI && i + 1 < T) {
#pragma unroll
            for (int j = 0; j < 4; ++j) kk[j] = nk[j], qq[j] = nq[j], dk[j] = nd[j], vv[j] = nv[j];
            b = nb;
        }
    }
    kda_store_state(x, Sp);
}

// ------------------------------------------------------------------ whole KDA layer step
// KDAAttention.__call__ for one token (attention_kda.py:94-115): the recurrence block also
// builds its inputs from the projection outputs: the short convolutions with SiLU
// (ops.py:46-60) of q, k (all 128 channels of the head) and v (the block's 32 columns),
// the L2 normalisation of q and k (ops.py:31-33, eps 1e-6), the decay gate
// lower_bound * sigmoid(exp(A_log[h]) * (f_b(f_a x) + dt_bias)) and beta = sigmoid(b x).
// The convolution states are read from conv_in and written to conv_out (distinct buffers),
// so no block reads a state another block rewrites.
struct KdaStepArgs {
    const float *q_raw, *k_raw, *v_raw;     // [P] projections of x
    const float *fb, *b_raw;                 // [P] f_b(f_a x), [H] b x
    const float *q_conv, *k_conv, *v_conv;   // [P, kc]
    const float *conv_in;                    // [3, kc - 1, P] (q, k, v), oldest first
    float *conv_out;                         // [3, kc - 1, P]
    const float *A_log, *dt_bias;            // [>= H], [P]
    float lower, scale;
    float *S;                                // [H, 128, 128] fp32, in place
    const float *og;                         // [P] g_proj x (the output gate logits)
    float *o;                                // [P] fp32: o * sigmoid(og)
    float *hss;                              // [H, 4] sum of o^2 over each block's 32 columns
    int H, kc;
};

__global__ __launch_bounds__(256) void kda_step_kernel(KdaStepArgs a) {
    __shared__ float red[2][4][kKdaVS];
    __shared__ float qs[kKdaK], ks[kKdaK], gs[kKdaK], vsh[kKdaVS], nrm[4];
    constexpr int V = kKdaK, nvb = kKdaK / kKdaVS;
    const int h = blockIdx.x / nvb, vb = blockIdx.x % nvb;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, cg = t & 7, r = t >> 3;
    const int P = a.H * kKdaK, kc = a.kc;
    const int c0 = vb * kKdaVS + 4 * cg;
    float *Sp[4];
    float4 x[4];
    kda_load_state(a.S, h, V, c0, x, Sp);
    // q (threads 0..127) and k (128..255): convolution, SiLU, then the L2 norm of the head
    {
        const int m = t >> 7, ch = h * kKdaK + (t & 127);
        const float *cw = (m ? a.k_conv : a.q_conv) + static_cast<int64_t>(ch) * kc;
        const float *cin = a.conv_in + static_cast<int64_t>(m) * (kc - 1) * P + ch;
        const float xr = (m ? a.k_raw : a.q_raw)[ch];
        float y = 0.f;
        for (int j = 0; j < kc - 1; ++j) y = fmaf(cw[j], cin[static_cast<int64_t>(j) * P], y);
        y = fmaf(cw[kc - 1], xr, y);
        y = y / (1.0f + expf(-y));
        if (vb == 0) {
            float *cout = a.conv_out + static_cast<int64_t>(m) * (kc - 1) * P + ch;
            for (int j = 0; j < kc - 2; ++j) cout[static_cast<int64_t>(j) * P] = cin[static_cast<int64_t>(j + 1) * P];
            cout[static_cast<int64_t>(kc - 2) * P] = xr;
        }
        const float ss = wave_sum_all(y * y);
        if (lane == 0) nrm[wave] = ss;
        __syncthreads();
        const float n = m ? nrm[2] + nrm[3] : nrm[0] + nrm[1];
        const float yn = y / sqrtf(n + 1e-6f);
        if (m == 0)
            qs[t] = yn * a.scale;
        else
            ks[t - 128] = yn;
    }
    // v for this block's columns (and their convolution states), the decay gate, beta
    if (t < kKdaVS) {
        const int ch = h * kKdaK + vb * kKdaVS + t;
        const float *cw = a.v_conv + static_cast<int64_t>(ch) * kc;
        const float *cin = a.conv_in + static_cast<int64_t>(2) * (kc - 1) * P + ch;
        const float xr = a.v_raw[ch];
        float y = 0.f;
        for (int j = 0; j < kc - 1; ++j) y = fmaf(cw[j], cin[static_cast<int64_t>(j) * P], y);
        y = fmaf(cw[kc - 1], xr, y);
        vsh[t] = y / (1.0f + expf(-y));
        float *cout = a.conv_out + static_cast<int64_t>(2) * (kc - 1) * P + ch;
        for (int j = 0; j < kc - 2; ++j) cout[static_cast<int64_t>(j) * P] = cin[static_cast<int64_t>(j + 1) * P];
        cout[static_cast<int64_t>(kc - 2) * P] = xr;
    }
    if (t >= 128) {
        const int i = t - 128, ch = h * kKdaK + i;
        const float z = expf(a.A_log[h]) * (a.fb[ch] + a.dt_bias[ch]);
        gs[i] = a.lower / (1.0f + expf(-z));
    }
    const float b = 1.0f / (1.0f + expf(-a.b_raw[h]));
    __syncthreads();
    float kk[4], qq[4], dk[4], vv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        kk[j] = ks[r + 32 * j];
        qq[j] = qs[r + 32 * j];
        dk[j] = expf(gs[r + 32 * j]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) vv[c] = vsh[4 * cg + c];
    const float o = kda_apply(x, kk, qq, dk, vv, b, red);
    kda_store_state(x, Sp);
    // the block's share of the head's sum of squares (for the gated RMSNorm), and o gated
    if (t < kKdaVS) {
        float ss = o * o;
        ss += __shfl_xor(ss, 1);
        ss += __shfl_xor(ss, 2);
        ss += __shfl_xor(ss, 4);
        ss += __shfl_xor(ss, 8);
        ss += __shfl_xor(ss, 16);
        if (t == 0) a.hss[h * nvb + vb] = ss;
        const int64_t c = static_cast<int64_t>(h) * V + vb * kKdaVS + t;
        a.o[c] = o / (1.0f + expf(-a.og[c]));
    }
}

}  // namespace
}  // namespace k3

using namespace k3;

static int kda_recurrent_impl(const void *q, const void *k, const void *v, const void *g, const void *beta,
                              int in_dtype, float *state, void *out, int out_dtype, int64_t T, int64_t qk_heads,
                              int64_t v_heads, int64_t key_dim, int64_t value_dim, float scale, void *stream) {
    if (!q || !k || !v || !g || !beta || !state || !out) return set_error(K3_ERR_NULL, "kda recurrence: null pointer");
    if (in_dtype != K3_F32 && in_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "kda recurrence: in_dtype %d", in_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "kda recurrence: out_dtype %d", out_dtype);
    if (key_dim != kKdaK)
        return set_error(K3_ERR_SHAPE, "kda recurrence: key_dim=%lld; the kernel takes %d", (long long)key_dim, kKdaK);
    if (value_dim <= 0 || value_dim % kKdaVS || value_dim > 4096)
        return set_error(K3_ERR_SHAPE, "kda recurrence: value_dim=%lld must be a positive multiple of %d, <= 4096",
                         (long long)value_dim, kKdaVS);
    if (qk_heads <= 0 || v_heads <= 0 || v_heads % qk_heads || v_heads > (1 << 20))
        return set_error(K3_ERR_SHAPE, "kda recurrence: v_heads=%lld must be a positive multiple of qk_heads=%lld",
                         (long long)v_heads, (long long)qk_heads);
    if (T <= 0 || T > (1 << 24)) return set_error(K3_ERR_SHAPE, "kda recurrence: T=%lld", (long long)T);
    if (!aligned16(state)) return set_error(K3_ERR_ALIGN, "kda recurrence: the state must be 16-byte aligned");
    KdaArgs a{};
    a.q = q, a.k = k, a.v = v, a.g = g, a.beta = beta;
    a.in_bf16 = in_dtype == K3_BF16;
    a.S = state;
    a.out = out;
    a.out_bf16 = out_dtype == K3_BF16;
    a.HV = static_cast<int>(v_heads);
    a.G = static_cast<int>(v_heads / qk_heads);
    a.V = static_cast<int>(value_dim);
    a.T = static_cast<int>(T);
    a.scale = scale;
    const int64_t blocks = v_heads * (value_dim / kKdaVS);
    if (T == 1)
        kda_decode_kernel<false><<<dim3(static_cast<unsigned>(blocks)), 256, 0, static_cast<hipStream_t>(stream)>>>(a);
    else
        kda_decode_kernel<true><<<dim3(static_cast<unsigned>(blocks)), 256, 0, static_cast<hipStream_t>(stream)>>>(a);
    return check_hip(hipGetLastError(), "kda recurrence launch");
}

extern "C" int k3_kda_recurrent_decode(const void *q, const void *k, const void *v, const void *g, const void *beta,
                                       int in_dtype, float *state, void *out, int out_dtype, int64_t qk_heads,
                                       int64_t v_heads, int64_t key_dim, int64_t value_dim, float scale,
                                       void *stream) {
    return kda_recurrent_impl(q, k, v, g, beta, in_dtype, state, out, out_dtype, 1, qk_heads, v_heads, key_dim,
                              value_dim, scale, stream);
}

extern "C" int k3_kda_recurrent(const void *q, const void *k, const void *v, const void *g, const void *beta,
                                int in_dtype, float *state, void *out, int out_dtype, int64_t T, int64_t qk_heads,
                                int64_t v_heads, int64_t key_dim, int64_t value_dim, float scale, void *stream) {
    return kda_recurrent_impl(q, k, v, g, beta, in_dtype, state, out, out_dtype, T, qk_heads, v_heads, key_dim,
                              value_dim, scale, stream);
}

namespace {
struct KdaStepWs {
    size_t q, k, v, og, fa, b, fb, o, hss, total;
};
KdaStepWs kda_step_ws(int64_t H) {
    const size_t P = static_cast<size_t>(H) * kKdaK;
    KdaStepWs L{};
    size_t off = 0;
    auto take = [&](size_t n) { const size_t at = off; off += (n * 4 + 255) & ~size_t(255); return at; };
    L.q = take(P), L.k = take(P), L.v = take(P), L.og = take(P), L.fa = take(kKdaK), L.b = take(H), L.fb = take(P);
    L.o = take(P);
    L.hss = take(static_cast<size_t>(H) * (kKdaK / kKdaVS));
    L.total = off;
    return L;
}
}  // namespace

extern "C" int64_t k3_kda_step_workspace_size(int64_t heads) { return static_cast<int64_t>(kda_step_ws(heads).total); }

extern "C" int k3_kda_step_decode(const void *x, int x_dtype, const void *q_proj, const void *k_proj,
                                  const void *v_proj, const void *g_proj, const void *o_proj, const void *f_a,
                                  const void *f_b, const void *b_proj, const float *q_conv, const float *k_conv,
                                  const float *v_conv, const float *conv_in, float *conv_out, const float *o_norm,
                                  const float *A_log, const float *dt_bias, float *state, void *out, int out_dtype,
                                  int64_t hidden, int64_t heads, int64_t head_dim, int64_t conv_size,
                                  float gate_lower_bound, float eps, void *workspace, int64_t workspace_bytes,
                                  void *stream) {
    if (!x || !q_proj || !k_proj || !v_proj || !g_proj || !o_proj || !f_a || !f_b || !b_proj || !q_conv || !k_conv ||
        !v_conv || !conv_in || !conv_out || !o_norm || !A_log || !dt_bias || !state || !out || !workspace)
        return set_error(K3_ERR_NULL, "kda step: null pointer");
    if (x_dtype != K3_F32 && x_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "kda step: x_dtype %d", x_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "kda step: out_dtype %d", out_dtype);
    if (head_dim != kKdaK) return set_error(K3_ERR_SHAPE, "kda step: head_dim=%lld; the kernels take %d",
                                            (long long)head_dim, kKdaK);
    const int64_t P = heads * head_dim;
    if (heads <= 0 || P > kMaxWidth || hidden <= 0 || hidden % 8 || hidden > kMaxWidth)
        return set_error(K3_ERR_SHAPE, "kda step: heads*head_dim and hidden must be <= %d (hidden a multiple of 8)",
                         kMaxWidth);
    if (conv_size < 2 || conv_size > 8) return set_error(K3_ERR_SHAPE, "kda step: conv_size=%lld", (long long)conv_size);
    if (conv_in == conv_out) return set_error(K3_ERR_SHAPE, "kda step: conv_in and conv_out must be distinct buffers");
    if (!aligned16(x) || !aligned16(q_proj) || !aligned16(k_proj) || !aligned16(v_proj) || !aligned16(g_proj) ||
        !aligned16(o_proj) || !aligned16(f_a) || !aligned16(f_b) || !aligned16(b_proj) || !aligned16(o_norm) ||
        !aligned16(state) || !aligned16(workspace))
        return set_error(K3_ERR_ALIGN, "kda step: vectors, weights, state and workspace must be 16-byte aligned");
    if (P * hidden * 2 >= (1ll << 31)) return set_error(K3_ERR_SHAPE, "kda step: a weight matrix exceeds 2 GiB");
    const KdaStepWs L = kda_step_ws(heads);
    if (workspace_bytes < static_cast<int64_t>(L.total))
        return set_error(K3_ERR_WORKSPACE, "kda step: workspace %lld < %zu bytes", (long long)workspace_bytes, L.total);
    char *ws = static_cast<char *>(workspace);
    float *wq = reinterpret_cast<float *>(ws + L.q), *wk = reinterpret_cast<float *>(ws + L.k);
    float *wv = reinterpret_cast<float *>(ws + L.v), *wog = reinterpret_cast<float *>(ws + L.og);
    float *wfa = reinterpret_cast<float *>(ws + L.fa), *wb = reinterpret_cast<float *>(ws + L.b);
    float *wfb = reinterpret_cast<float *>(ws + L.fb), *wo = reinterpret_cast<float *>(ws + L.o);
    float *whss = reinterpret_cast<float *>(ws + L.hss);
    auto st = static_cast<hipStream_t>(stream);
    // K1: rows of q, k, v, g, f_a and b against x
    RowsArgs a1{};
    a1.x = x, a1.x_bf16 = x_dtype == K3_BF16, a1.K = static_cast<int>(hidden);
    const void *w1[6] = {q_proj, k_proj, v_proj, g_proj, f_a, b_proj};
    float *y1[6] = {wq, wk, wv, wog, wfa, wb};
    const int n1[6] = {static_cast<int>(P), static_cast<int>(P), static_cast<int>(P), static_cast<int>(P), kKdaK,
                       static_cast<int>(heads)};
    for (int i = 0; i < 6; ++i) a1.w[i] = static_cast<const uint16_t *>(w1[i]), a1.N[i] = n1[i], a1.y[i] = y1[i];
    int rc = launch_rows<kModeX>(a1, st);
    if (rc) return rc;
    // K2: rows of f_b against f_a x
    RowsArgs a2{};
    a2.o = wfa, a2.K = kKdaK;
    a2.w[0] = static_cast<const uint16_t *>(f_b), a2.N[0] = static_cast<int>(P), a2.y[0] = wfb;
    rc = launch_rows<kModeGate>(a2, st);
    if (rc) return rc;
    // K3: convolutions, norms, gate and the recurrence
    KdaStepArgs k{};
    k.q_raw = wq, k.k_raw = wk, k.v_raw = wv, k.fb = wfb, k.b_raw = wb;
    k.q_conv = q_conv, k.k_conv = k_conv, k.v_conv = v_conv, k.conv_in = conv_in, k.conv_out = conv_out;
    k.A_log = A_log, k.dt_bias = dt_bias, k.lower = gate_lower_bound, k.scale = 1.0f / sqrtf(static_cast<float>(kKdaK));
    k.S = state, k.og = wog, k.o = wo, k.hss = whss, k.H = static_cast<int>(heads), k.kc = static_cast<int>(conv_size);
    kda_step_kernel<<<dim3(static_cast<unsigned>(heads * (kKdaK / kKdaVS))), 256, 0, st>>>(k);
    rc = check_hip(hipGetLastError(), "kda step: recurrence launch");
    if (rc) return rc;
    // K4: rows of o_proj against the gated heads scaled by their RMS norms, in the persistent
    // row form (one block per CU stages the 48 KB vector once): measured faster for this
    // launch, while K1 measured slower in that form
    RowsArgs a4{};
    a4.o = wo, a4.gl = whss, a4.nw = o_norm, a4.eps = eps, a4.K = static_cast<int>(P);
    a4.w[0] = static_cast<const uint16_t *>(o_proj), a4.N[0] = static_cast<int>(hidden);
    a4.out = out, a4.out_bf16 = out_dtype == K3_BF16;
    return launch_rows_loop<kModeHeadNorm>(a4, st);
}
