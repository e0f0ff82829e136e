// One decode token through a whole MLA layer at batch 1: the projections on either side
// of the absorbed attention core, the latent-cache append and the output gate.
//
// Reference: MLAAttention.__call__ (air_llm/models/kimi_k3/attention_mla.py:168-216):
//   q   = rmsnorm(x @ q_a.T, q_a_layernorm) @ q_b.T                  -> [H, nope + rope]
//   ckv = x @ kv_a.T;  c_new = rmsnorm(ckv[:r], kv_a_layernorm);  r_new = ckv[r:]
//   cache.append(c_new, r_new)                                      (attention_mla.py:89-108)
//   o   = absorbed attention core over the cache                     (attention_mla.py:193-212)
//   o   = o * sigmoid(x @ g_proj.T)  (mla_use_output_gate);  out = o @ o_proj.T
//
// Six stream-ordered launches, no host synchronisation:
//   S1  rows of q_a, kv_a and g_proj against x (one grid, three block ranges);
//   S2  rows of q_b against the normalised q_a output (every block normalises the 1536-wide
//       vector itself, so no launch is spent on it), and one block that normalises the kv
//       latent and writes the new cache row (bf16) at position pos;
//   core  the absorbed core of k3_mla_decode_absorbed (three launches) over the pos + 1
//       cache rows, its last launch multiplying o by sigmoid(gate) as it writes it;
//   S3  rows of o_proj against the gated o.
// Every row kernel issues its weight rows first, then stages its fp32 input vector in LDS
// (K floats), then reduces: a lane takes 16-byte chunks (8 bf16) l, l + 64, ... of a row.
#include <algorithm>

#include "k3_common.h"

namespace k3 {
namespace {

enum { kModeX = 0, kModeNorm = 1, kModeGate = 2 };
constexpr int kMaxWidth = 12288;  // input vector width (fp32 in LDS: 48 KB)

struct RowsArgs {
    const void *x;            // kModeX: [K] bf16 or fp32
    int x_bf16;
    const float *src, *nw;    // kModeNorm: v = src * rsqrt(mean(src^2) + eps) * nw
    float eps;
    const float *o, *gl;      // kModeGate: v = o * sigmoid(gl) (gl null: v = o)
    int K;
    const uint16_t *w[3];     // up to three bf16 row sets [N, K] sharing v
    int N[3];
    int blocks[3];
    float *y[3];              // fp32 outputs [N] (kModeGate: y[0] unused, out below)
    void *out;                // kModeGate: [N] fp32 or bf16
    int out_bf16;
    // kModeNorm, last block: the cache append
    const float *ckv, *kvw;   // ckv [r + rope] fp32, kv_a_layernorm [r]
    uint16_t *lat_row, *rot_row;
    int r, rope, append;
};

__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum_all(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float t = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return t;
}

// v (fp32, K values) into LDS; ends with a block barrier
template <int MODE>
__device__ __forceinline__ void stage_vector(const RowsArgs &a, float *vs, float *red) {
    const int K = a.K;
    if (MODE == kModeX) {
        if (a.x_bf16) {
            const uint4 *x8 = static_cast<const uint4 *>(a.x);
            for (int c = threadIdx.x; c < K / 8; c += 256) {
                const uint4 q = x8[c];
                const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    vs[8 * c + 2 * i] = __uint_as_float(d[i] << 16);
                    vs[8 * c + 2 * i + 1] = __uint_as_float(d[i] & 0xffff0000u);
                }
            }
        } else {
            const float4 *x4 = static_cast<const float4 *>(a.x);
            for (int c = threadIdx.x; c < K / 4; c += 256) reinterpret_cast<float4 *>(vs)[c] = x4[c];
        }
    } else if (MODE == kModeNorm) {
        float ss = 0.f;
        for (int c = threadIdx.x; c < K / 4; c += 256) {
            const float4 s = reinterpret_cast<const float4 *>(a.src)[c];
            ss = fmaf(s.x, s.x, fmaf(s.y, s.y, fmaf(s.z, s.z, fmaf(s.w, s.w, ss))));
            reinterpret_cast<float4 *>(vs)[c] = s;
        }
        const float rs = 1.0f / sqrtf(block_sum(ss, red) / static_cast<float>(K) + a.eps);
        for (int c = threadIdx.x; c < K / 4; c += 256) {
            const float4 g = reinterpret_cast<const float4 *>(a.nw)[c];
            float4 v = reinterpret_cast<float4 *>(vs)[c];
            v.x = v.x * rs * g.x, v.y = v.y * rs * g.y, v.z = v.z * rs * g.z, v.w = v.w * rs * g.w;
            reinterpret_cast<float4 *>(vs)[c] = v;
        }
    } else {
        for (int c = threadIdx.x; c < K / 4; c += 256) {
            float4 v = reinterpret_cast<const float4 *>(a.o)[c];
            if (a.gl) {
                const float4 g = reinterpret_cast<const float4 *>(a.gl)[c];
                v.x /= 1.0f + expf(-g.x), v.y /= 1.0f + expf(-g.y), v.z /= 1.0f + expf(-g.z),
                    v.w /= 1.0f + expf(-g.w);
            }
            reinterpret_cast<float4 *>(vs)[c] = v;
        }
    }
    __syncthreads();
}

// c_new = rmsnorm(ckv[:r]) * kv_a_layernorm -> lat_row (bf16); rot_row = bf16(ckv[r:])
__device__ void append_row(const RowsArgs &a, float *red) {
    float ss = 0.f;
    for (int j = threadIdx.x; j < a.r; j += 256) ss = fmaf(a.ckv[j], a.ckv[j], ss);
    const float rs = 1.0f / sqrtf(block_sum(ss, red) / static_cast<float>(a.r) + a.eps);
    for (int j = threadIdx.x; j < a.r; j += 256) a.lat_row[j] = f32_to_bf16(a.ckv[j] * rs * a.kvw[j]);
    for (int j = threadIdx.x; j < a.rope; j += 256) a.rot_row[j] = f32_to_bf16(a.ckv[a.r + j]);
}

// 8 bf16 weights . 8 fp32 values
__device__ __forceinline__ float dot8_bf16_f32(uint4 w, float4 v0, float4 v1, float acc) {
    acc = fmaf(__uint_as_float(w.x << 16), v0.x, acc);
    acc = fmaf(__uint_as_float(w.x & 0xffff0000u), v0.y, acc);
    acc = fmaf(__uint_as_float(w.y << 16), v0.z, acc);
    acc = fmaf(__uint_as_float(w.y & 0xffff0000u), v0.w, acc);
    acc = fmaf(__uint_as_float(w.z << 16), v1.x, acc);
    acc = fmaf(__uint_as_float(w.z & 0xffff0000u), v1.y, acc);
    acc = fmaf(__uint_as_float(w.w << 16), v1.z, acc);
    acc = fmaf(__uint_as_float(w.w & 0xffff0000u), v1.w, acc);
    return acc;
}

// Block: 4 waves x R rows of one row set; CH 16-byte chunks per lane per row.
template <int MODE, int CH, int R>
__global__ __launch_bounds__(256) void step_rows_kernel(RowsArgs a) {
    extern __shared__ float vs[];
    __shared__ float red[4];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (MODE == kModeNorm && a.append && static_cast<int>(blockIdx.x) == static_cast<int>(gridDim.x) - 1) {
        append_row(a, red);
        return;
    }
    int b = blockIdx.x, s = 0;
    while (s < 2 && b >= a.blocks[s]) b -= a.blocks[s++];
    const int N = a.N[s], K = a.K, nch = K >> 3;
    const uint32_t rowb = static_cast<uint32_t>(K) * 2u;
    const int n0 = (b * 4 + wave) * R;
    const auto rw = make_rsrc(a.w[s], static_cast<uint32_t>(N) * rowb);
    // 1. the wave's rows
    uint4 wr[R][CH];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int c = u * 64 + lane, n = n0 + r;
            wr[r][u] = buf_load16(rw, (n < N && c < nch) ? static_cast<uint32_t>(n) * rowb + c * 16u : kOobOffset);
        }
    // 2. the input vector
    stage_vector<MODE>(a, vs, red);
    // 3. row dots
    const float4 *v4 = reinterpret_cast<const float4 *>(vs);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int c = u * 64 + lane;
            if (c < nch) {
                if (u & 1)
                    acc1 = dot8_bf16_f32(wr[r][u], v4[2 * c], v4[2 * c + 1], acc1);
                else
                    acc0 = dot8_bf16_f32(wr[r][u], v4[2 * c], v4[2 * c + 1], acc0);
            }
        }
        const float t = wave_sum_to_lane63(acc0 + acc1);
        const int n = n0 + r;
        if (lane == 63 && n < N) {
            if (MODE == kModeGate) {
                if (a.out_bf16)
                    static_cast<uint16_t *>(a.out)[n] = f32_to_bf16(t);
                else
                    static_cast<float *>(a.out)[n] = t;
            } else {
                a.y[s][n] = t;
            }
        }
    }
}

template <int MODE, int CH>
int launch_rows_ch(RowsArgs &a, hipStream_t st) {
    constexpr int R = CH >= 16 ? 1 : (CH >= 8 ? 2 : (CH >= 4 ? 4 : 8));
    int total = 0;
    for (int s = 0; s < 3; ++s) {
        a.blocks[s] = a.w[s] ? static_cast<int>(cdiv(a.N[s], 4 * R)) : 0;
        total += a.blocks[s];
    }
    if (MODE == kModeNorm && a.append) ++total;
    step_rows_kernel<MODE, CH, R><<<dim3(static_cast<unsigned>(total)), 256, static_cast<size_t>(a.K) * 4, st>>>(a);
    return check_hip(hipGetLastError(), "mla step rows");
}

template <int MODE>
int launch_rows(RowsArgs &a, hipStream_t st) {
    const int ch = static_cast<int>(cdiv(a.K / 8, 64));
    if (ch <= 1) return launch_rows_ch<MODE, 1>(a, st);
    if (ch <= 2) return launch_rows_ch<MODE, 2>(a, st);
    if (ch <= 4) return launch_rows_ch<MODE, 4>(a, st);
    if (ch <= 8) return launch_rows_ch<MODE, 8>(a, st);
    if (ch <= 16) return launch_rows_ch<MODE, 16>(a, st);
    if (ch <= 24) return launch_rows_ch<MODE, 24>(a, st);
    return set_error(K3_ERR_SHAPE, "mla step: input width %d above %d", a.K, kMaxWidth);
}

size_t up256(size_t v) { return (v + 255) & ~size_t(255); }

struct StepWs {
    size_t qa, ckv, gl, q, o, core, total;
};

StepWs step_ws_layout(int64_t hidden, int64_t ql, int64_t H, int64_t nope, int64_t rope, int64_t v, int64_t r,
                      int64_t T) {
    StepWs L{};
    size_t off = 0;
    L.qa = off, off += up256(ql * 4);
    L.ckv = off, off += up256((r + rope) * 4);
    L.gl = off, off += up256(H * v * 4);
    L.q = off, off += up256(H * (nope + rope) * 4);
    L.o = off, off += up256(H * v * 4);
    L.core = off, off += static_cast<size_t>(k3_mla_workspace_size(H, T));
    L.total = off;
    (void)hidden;
    return L;
}

}  // namespace
}  // namespace k3

using namespace k3;

extern "C" int64_t k3_mla_step_workspace_size(int64_t hidden, int64_t q_lora_rank, int64_t heads, int64_t nope_dim,
                                              int64_t rope_dim, int64_t v_dim, int64_t kv_lora_rank, int64_t T) {
    return static_cast<int64_t>(
        step_ws_layout(hidden, q_lora_rank, heads, nope_dim, rope_dim, v_dim, kv_lora_rank, T).total);
}

extern "C" int k3_mla_step_decode(const void *x, int x_dtype, const void *q_a, const float *q_a_norm, const void *q_b,
                                  const void *kv_a, const float *kv_a_norm, const void *w_uk, const void *w_uv,
                                  const void *g_proj, const void *o_proj, void *lat, int64_t ld_lat, void *rot,
                                  int64_t ld_rot, int64_t cache_rows, int64_t pos, float eps, float scale, void *out,
                                  int out_dtype,
                                  int64_t hidden, int64_t q_lora_rank, int64_t heads, int64_t nope_dim,
                                  int64_t rope_dim, int64_t v_dim, int64_t kv_lora_rank, void *workspace,
                                  int64_t workspace_bytes, void *stream) {
    if (!x || !q_a || !q_a_norm || !q_b || !kv_a || !kv_a_norm || !w_uk || !w_uv || !o_proj || !lat || !rot || !out ||
        !workspace)
        return set_error(K3_ERR_NULL, "mla step: null pointer");
    if (x_dtype != K3_F32 && x_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "mla step: x_dtype %d", x_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "mla step: out_dtype %d", out_dtype);
    const int64_t qhd = nope_dim + rope_dim, hv = heads * v_dim;
    if (hidden <= 0 || hidden % 8 || q_lora_rank <= 0 || q_lora_rank % 8 || hv <= 0 || hv % 8 ||
        hidden > kMaxWidth || q_lora_rank > kMaxWidth || hv > kMaxWidth || kv_lora_rank % 4 || rope_dim % 4)
        return set_error(K3_ERR_SHAPE, "mla step: hidden, q_lora_rank and heads*v must be multiples of 8, <= %d",
                         kMaxWidth);
    if (pos < 0 || pos >= cache_rows)
        return set_error(K3_ERR_SHAPE, "mla step: position %lld outside the cache's %lld rows", (long long)pos,
                         (long long)cache_rows);
    if (!aligned16(x) || !aligned16(q_a) || !aligned16(q_b) || !aligned16(kv_a) || !aligned16(o_proj) ||
        (g_proj && !aligned16(g_proj)) || !aligned16(q_a_norm) || !aligned16(kv_a_norm) || !aligned16(workspace))
        return set_error(K3_ERR_ALIGN, "mla step: vectors, weights and workspace must be 16-byte aligned");
    if (heads * qhd * q_lora_rank * 2 >= (1ll << 31) || hidden * hv * 2 >= (1ll << 31) ||
        q_lora_rank * hidden * 2 >= (1ll << 31))
        return set_error(K3_ERR_SHAPE, "mla step: a weight matrix exceeds 2 GiB");
    const int64_t T = pos + 1;
    const StepWs L = step_ws_layout(hidden, q_lora_rank, heads, nope_dim, rope_dim, v_dim, kv_lora_rank, T);
    if (workspace_bytes < static_cast<int64_t>(L.total))
        return set_error(K3_ERR_WORKSPACE, "mla step: workspace %lld < %zu bytes", (long long)workspace_bytes, L.total);
    char *ws = static_cast<char *>(workspace);
    float *qa = reinterpret_cast<float *>(ws + L.qa), *ckv = reinterpret_cast<float *>(ws + L.ckv);
    float *gl = reinterpret_cast<float *>(ws + L.gl), *q = reinterpret_cast<float *>(ws + L.q);
    float *o = reinterpret_cast<float *>(ws + L.o);
    auto st = static_cast<hipStream_t>(stream);
    // S1: q_a, kv_a, g_proj rows against x
    RowsArgs a{};
    a.x = x;
    a.x_bf16 = x_dtype == K3_BF16;
    a.K = static_cast<int>(hidden);
    a.w[0] = static_cast<const uint16_t *>(q_a), a.N[0] = static_cast<int>(q_lora_rank), a.y[0] = qa;
    a.w[1] = static_cast<const uint16_t *>(kv_a), a.N[1] = static_cast<int>(kv_lora_rank + rope_dim), a.y[1] = ckv;
    a.w[2] = static_cast<const uint16_t *>(g_proj), a.N[2] = g_proj ? static_cast<int>(hv) : 0, a.y[2] = gl;
    int rc = launch_rows<kModeX>(a, st);
    if (rc) return rc;
    // S2: q_b rows against the normalised q_a output; the cache row
    RowsArgs b{};
    b.src = qa, b.nw = q_a_norm, b.eps = eps, b.K = static_cast<int>(q_lora_rank);
    b.w[0] = static_cast<const uint16_t *>(q_b), b.N[0] = static_cast<int>(heads * qhd), b.y[0] = q;
    b.ckv = ckv, b.kvw = kv_a_norm;
    b.lat_row = static_cast<uint16_t *>(lat) + pos * ld_lat;
    b.rot_row = static_cast<uint16_t *>(rot) + pos * ld_rot;
    b.r = static_cast<int>(kv_lora_rank), b.rope = static_cast<int>(rope_dim), b.append = 1;
    rc = launch_rows<kModeNorm>(b, st);
    if (rc) return rc;
    // core over the pos + 1 cache rows
    rc = mla_decode_core(q, q + nope_dim, qhd, qhd, K3_F32, w_uk, w_uv, lat, ld_lat, rot, ld_rot, T, heads,
                         kv_lora_rank, rope_dim, nope_dim, v_dim, scale, o, K3_F32, v_dim, g_proj ? gl : nullptr,
                         ws + L.core, workspace_bytes - static_cast<int64_t>(L.core), stream);
    if (rc) return rc;
    // S3: o_proj rows against the gated o
    RowsArgs c{};
    c.o = o, c.gl = nullptr, c.K = static_cast<int>(hv);
    c.w[0] = static_cast<const uint16_t *>(o_proj), c.N[0] = static_cast<int>(hidden);
    c.out = out, c.out_bf16 = out_dtype == K3_BF16;
    return launch_rows<kModeGate>(c, st);
}
