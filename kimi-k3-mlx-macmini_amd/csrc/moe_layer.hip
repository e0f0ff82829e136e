// Routed MoE layer decode at batch 1 (router + top-k + routed experts + shared expert +
// weighted combine), four stream-ordered launches with no host synchronisation.
//
// Reference: LatentMoE.route / __call__ / shared_forward (air_llm/models/kimi_k3/moe.py:65-132,
// k3ref/layers.py:214-261).  The reference materialises the routing on the host
// (np_indices, moe.py:135-138) and loops over experts serially with an mx.eval per expert.
// Here the routing never leaves the GPU:
//
//   K1  router logits (bf16 [E, H] x bf16/fp32 x)          -> ws.logits[E]
//       shared expert gate/up rows (bf16) + activation       -> ws.shared_act[Is]
//   R   one block: softmax/sigmoid + rank-based top-k of the E logits, the router
//       records for the caller, and the k selected experts' weight pointers
//   K2  routed gate/up rows of the k selected experts       -> ws.act[k][I]
//       (expert weights through a device table of pointers, so all E experts stay
//       resident and each selected expert's bytes are read exactly once)
//       shared down rows (bf16 [H, Is] x shared_act)        -> ws.yshared[H]
//   K3  per output row: the k routed down rows (MXFP4) against ws.act[j], combined in a
//       fixed order y = yshared + sum_j w_j * down_j      -> out[H]
#include <algorithm>

#include "moe_common.h"
#include "mxfp4_dot.h"

namespace k3 {

// Workspace layout (byte offsets computed on the host, see layer_ws_layout).
struct LayerWs {
    float *logits;       // [E]
    float *scores;       // [E]  raw scores (softmax probabilities or sigmoid)
    float *corrected;    // [E]  selection scores (== scores for softmax)
    int32_t *topk_idx;   // [k]
    float *topk_w;       // [k]
    float *shared_act;   // [Is]
    float *act;          // [k][I]
    float *yshared;      // [H]
    uint64_t *sel_ptrs;  // [k][6] weight pointers of the selected experts
};

struct LayerArgs {
    const void *x;                 // [H]
    const uint16_t *router_w;      // [E, H] bf16
    const float *router_bias;      // [E] or null (sigmoid_bias routing)
    const uint64_t *table;         // [E][6] device pointers: gate p/s, up p/s, down p/s
    const uint16_t *sh_gate, *sh_up, *sh_down;  // bf16 [Is, H], [Is, H], [H, Is]; null: none
    void *out;                     // [H]
    LayerWs ws;
    int H, I, Is, E, k;
    int route_kind, renorm;
    float scaling;
    int act_kind;
    float beta, lbeta;
    int out_bf16;
    int k1_router_blocks;          // K1: blocks [0, k1_router_blocks) do router rows
    int k2_routed_blocks;          // K2: blocks [0, k2_routed_blocks) do routed gate/up
};

constexpr int kMaxTopK = 16;
constexpr int kMaxExperts = 1024;

// ------------------------------------------------------------------ bf16 row dots
// 8 bf16 weights . 8 bf16 activations
__device__ __forceinline__ float dot8(uint4 w, uint4 x, float acc) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.x), __builtin_bit_cast(bf16x2, x.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.y), __builtin_bit_cast(bf16x2, x.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.z), __builtin_bit_cast(bf16x2, x.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.w), __builtin_bit_cast(bf16x2, x.w), acc, false);
    return acc;
}
// 8 bf16 weights . 8 fp32 activations (exact widening of the weights, fp32 FMA)
__device__ __forceinline__ float dot8(uint4 w, float4 x0, float4 x1, float acc) {
    acc = fmaf(__uint_as_float(w.x << 16), x0.x, acc);
    acc = fmaf(__uint_as_float(w.x & 0xffff0000u), x0.y, acc);
    acc = fmaf(__uint_as_float(w.y << 16), x0.z, acc);
    acc = fmaf(__uint_as_float(w.y & 0xffff0000u), x0.w, acc);
    acc = fmaf(__uint_as_float(w.z << 16), x1.x, acc);
    acc = fmaf(__uint_as_float(w.z & 0xffff0000u), x1.y, acc);
    acc = fmaf(__uint_as_float(w.w << 16), x1.z, acc);
    acc = fmaf(__uint_as_float(w.w & 0xffff0000u), x1.w, acc);
    return acc;
}

// Plain (unswizzled) LDS activation row: chunk c = 8 elements (bf16: one uint4;
// fp32: two float4).  Lanes read consecutive chunks, which is conflict-free.
template <typename XT>
__device__ __forceinline__ float dot_chunk(uint4 w, const uint4 *xl, int c, float acc) {
    if constexpr (std::is_same<XT, uint16_t>::value) {
        return dot8(w, xl[c], acc);
    } else {
        const float4 *xf = reinterpret_cast<const float4 *>(xl);
        return dot8(w, xf[2 * c], xf[2 * c + 1], acc);
    }
}

template <typename XT>
__device__ __forceinline__ void stage_plain(uint4 *dst, const void *src, int n_elems) {
    const int chunks = n_elems * static_cast<int>(sizeof(XT)) / 16;
    const uint4 *s = static_cast<const uint4 *>(src);
    for (int c = threadIdx.x; c < chunks; c += blockDim.x) dst[c] = s[c];
}

// NR bf16 weight rows (K elements each, K % 8 == 0) against an LDS activation row, in two
// halves so callers can issue the weight stream before staging the activations:
// bf16_rows_load issues every row's loads, bf16_rows_dot consumes them (wave totals land
// in lane 63).  CH = chunks of 8 per lane (compile-time upper bound).
template <int CH, int NR>
__device__ __forceinline__ void bf16_rows_load(const __amdgpu_buffer_rsrc_t (&r)[NR], const uint32_t (&row_off)[NR],
                                               int K, const bool (&valid)[NR], uint4 (&w)[NR][CH]) {
    const int lane = threadIdx.x & 63;
    const int nch = K >> 3;
#pragma unroll
    for (int q = 0; q < NR; ++q)
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int c = u * 64 + lane;
            w[q][u] = buf_load16(r[q], (valid[q] && c < nch) ? row_off[q] + c * 16u : kOobOffset);
        }
}

template <typename XT, int CH, int NR>
__device__ __forceinline__ void bf16_rows_dot(const uint4 (&w)[NR][CH], int K, const uint4 *xl, float (&out)[NR]) {
    const int lane = threadIdx.x & 63;
    const int nch = K >> 3;
    float acc[NR][2];
#pragma unroll
    for (int q = 0; q < NR; ++q) acc[q][0] = acc[q][1] = 0.f;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
        const int c = u * 64 + lane;
        if (c < nch) {
#pragma unroll
            for (int q = 0; q < NR; ++q) acc[q][u & 1] = dot_chunk<XT>(w[q][u], xl, c, acc[q][u & 1]);
        }
    }
#pragma unroll
    for (int q = 0; q < NR; ++q) out[q] = wave_sum_to_lane63(acc[q][0] + acc[q][1]);
}

// A 64-bit pointer held in LDS or loaded per lane, made wave-uniform (SGPRs) so buffer
// resources built from it need no waterfall loop.
__device__ __forceinline__ const void *uniform_ptr(uint64_t p) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
    return reinterpret_cast<const void *>((static_cast<uint64_t>(hi) << 32) | lo);
}

// ------------------------------------------------------------------ routing
// One block of E threads rounded up to a multiple of 64 (E <= 1024).
// softmax:       scores = softmax(logits), selection on scores
// sigmoid_bias:  scores = sigmoid(logits), selection on scores + bias, weights from scores
// weights: optional renormalisation by (sum + 1e-20), then * scaling   (moe.py:65-76)
// Top-k is exact and deterministic with ties to the lower expert index, in two levels:
// every expert ranks itself inside its 64-expert group (64 broadcast LDS compares), the
// group's best k become candidates, and each candidate ranks itself among all candidates.
// The global top-k is always inside the union of the per-group top-k.
__device__ __forceinline__ float block_reduce(float v, float *red, bool is_max) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = is_max ? wave_max_all(v) : wave_sum_all(v);
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float r = red[0];
    for (int i = 1; i < nw; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
    __syncthreads();
    return r;
}

// (value, index) order: larger value first, then lower index
__device__ __forceinline__ bool outranks(float v, int j, float sel, int e) {
    return v > sel || (v == sel && j < e);
}

__global__ __launch_bounds__(1024) void layer_route(LayerArgs a) {
    __shared__ __align__(16) float sel_s[kMaxExperts];
    __shared__ float cand_v[kMaxExperts / 64 * kMaxTopK];
    __shared__ int cand_e[kMaxExperts / 64 * kMaxTopK];
    __shared__ float cand_s[kMaxExperts / 64 * kMaxTopK];
    __shared__ float red[16];
    __shared__ int32_t idx_s[kMaxTopK];
    __shared__ float w_s[kMaxTopK];
    const int e = threadIdx.x;
    const int groups = blockDim.x >> 6;
    const bool live = e < a.E;
    const float l = live ? a.ws.logits[e] : -INFINITY;
    float s;
    if (a.route_kind == K3_ROUTE_SOFTMAX) {
        const float mx = block_reduce(l, red, true);
        const float ex = live ? expf(l - mx) : 0.f;
        const float sum = block_reduce(ex, red, false);
        s = ex / sum;
    } else {
        s = 1.0f / (1.0f + expf(-l));
    }
    const float sel = (a.route_kind == K3_ROUTE_SIGMOID_BIAS && a.router_bias && live) ? s + a.router_bias[e] : s;
    sel_s[e] = live ? sel : -INFINITY;
    for (int c = threadIdx.x; c < groups * a.k; c += blockDim.x) {
        cand_v[c] = -INFINITY;
        cand_e[c] = 0x7fffffff;
    }
    __syncthreads();
    if (live) {
        a.ws.scores[e] = s;
        a.ws.corrected[e] = sel;
        // rank inside the 64-expert group
        const int g0 = e & ~63;
        const float4 *s4 = reinterpret_cast<const float4 *>(sel_s + g0);
        int rank = 0;
#pragma unroll
        for (int j4 = 0; j4 < 16; ++j4) {
            const float4 v = s4[j4];
            const int j = g0 + j4 * 4;
            rank += outranks(v.x, j, sel, e) + outranks(v.y, j + 1, sel, e) + outranks(v.z, j + 2, sel, e) +
                    outranks(v.w, j + 3, sel, e);
        }
        if (rank < a.k) {
            const int c = (e >> 6) * a.k + rank;
            cand_v[c] = sel;
            cand_e[c] = e;
            cand_s[c] = s;
        }
    }
    __syncthreads();
    const int nc = groups * a.k;
    for (int c = threadIdx.x; c < nc; c += blockDim.x) {
        const float v = cand_v[c];
        const int ce = cand_e[c];
        if (ce == 0x7fffffff) continue;
        int rank = 0;
        for (int d = 0; d < nc; ++d) rank += outranks(cand_v[d], cand_e[d], v, ce);
        if (rank < a.k) {
            idx_s[rank] = ce;
            w_s[rank] = cand_s[c];
        }
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        float wsum = lane < a.k ? w_s[lane] : 0.f;
        wsum = wave_sum_all(wsum);
        const float norm = (a.renorm && a.k > 1) ? 1.0f / (wsum + 1e-20f) : 1.0f;
        if (lane < a.k) {
            a.ws.topk_idx[lane] = idx_s[lane];
            a.ws.topk_w[lane] = w_s[lane] * norm * a.scaling;
        }
    }
    if (a.table && static_cast<int>(threadIdx.x) < a.k * 6) {
        const int j = threadIdx.x / 6, q = threadIdx.x % 6;
        a.ws.sel_ptrs[threadIdx.x] = a.table[static_cast<int64_t>(idx_s[j]) * 6 + q];
    }
}

// ------------------------------------------------------------------ K1
template <typename XT, int CHH>
__global__ __launch_bounds__(256) void layer_k1(LayerArgs a) {
    extern __shared__ uint4 smem[];
    uint4 *xl = smem;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const uint32_t row_bytes = static_cast<uint32_t>(a.H) * 2u;
    if (static_cast<int>(blockIdx.x) < a.k1_router_blocks) {
        const int e = blockIdx.x * 4 + wave;
        const __amdgpu_buffer_rsrc_t r[1] = {make_rsrc(a.router_w, static_cast<uint32_t>(a.E) * row_bytes)};
        const uint32_t off[1] = {static_cast<uint32_t>(e) * row_bytes};
        const bool v[1] = {e < a.E};
        uint4 w[1][CHH];
        bf16_rows_load<CHH, 1>(r, off, a.H, v, w);
        stage_plain<XT>(xl, a.x, a.H);
        __syncthreads();
        float t[1];
        bf16_rows_dot<XT, CHH, 1>(w, a.H, xl, t);
        if (lane == 63 && e < a.E) a.ws.logits[e] = t[0];
    } else {
        const int i = (blockIdx.x - a.k1_router_blocks) * 4 + wave;
        const __amdgpu_buffer_rsrc_t r[2] = {make_rsrc(a.sh_gate, static_cast<uint32_t>(a.Is) * row_bytes),
                                             make_rsrc(a.sh_up, static_cast<uint32_t>(a.Is) * row_bytes)};
        const uint32_t off[2] = {static_cast<uint32_t>(i) * row_bytes, static_cast<uint32_t>(i) * row_bytes};
        const bool v[2] = {i < a.Is, i < a.Is};
        uint4 w[2][CHH];
        bf16_rows_load<CHH, 2>(r, off, a.H, v, w);
        stage_plain<XT>(xl, a.x, a.H);
        __syncthreads();
        float gu[2];
        bf16_rows_dot<XT, CHH, 2>(w, a.H, xl, gu);
        if (lane == 63 && i < a.Is) a.ws.shared_act[i] = act_fn(gu[0], gu[1], a.act_kind, a.beta, a.lbeta);
    }
}

// ------------------------------------------------------------------ K2
constexpr int kK2Pairs = 2;  // routed (gate, up) row pairs per wave

template <typename XT, int GA, int CHI>
__global__ __launch_bounds__(256) void layer_k2(LayerArgs a) {
    extern __shared__ uint4 smem[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (static_cast<int>(blockIdx.x) < a.k2_routed_blocks) {
        // routed gate/up: kK2Pairs row pairs (slot j, row i) per wave
        constexpr int CPGX = XTile<XT>::kChunks;
        const int GH = a.H >> 5;
        const uint32_t rowA = static_cast<uint32_t>(a.H >> 1);
        uint4 wg_[kK2Pairs][GA], wu_[kK2Pairs][GA];
        uint32_t sg_[kK2Pairs][GA], su_[kK2Pairs][GA];
        int jj[kK2Pairs], ii[kK2Pairs];
        bool vv[kK2Pairs];
#pragma unroll
        for (int p = 0; p < kK2Pairs; ++p) {
            const int pair = (blockIdx.x * 4 + wave) * kK2Pairs + p;
            const int j = pair / a.I, i = pair % a.I;
            const bool v = j < a.k;
            jj[p] = j, ii[p] = i, vv[p] = v;
            const uint64_t *t = a.ws.sel_ptrs + (v ? j : 0) * 6;
            const auto rg = make_rsrc(uniform_ptr(t[0]), static_cast<uint32_t>(a.I) * rowA);
            const auto rgs = make_rsrc(uniform_ptr(t[1]), static_cast<uint32_t>(a.I * GH));
            const auto ru = make_rsrc(uniform_ptr(t[2]), static_cast<uint32_t>(a.I) * rowA);
            const auto rus = make_rsrc(uniform_ptr(t[3]), static_cast<uint32_t>(a.I * GH));
            const uint32_t so = static_cast<uint32_t>(i * GH);
#pragma unroll
            for (int u = 0; u < GA; ++u) {
                const int g = u * 64 + lane;
                const bool ok = v && g < GH;
                const uint32_t off = ok ? static_cast<uint32_t>(i) * rowA + g * 16u : kOobOffset;
                const uint32_t soff = ok ? scale_dword_off(so, g) : kOobOffset;
                wg_[p][u] = buf_load16(rg, off);
                wu_[p][u] = buf_load16(ru, off);
                sg_[p][u] = buf_load4(rgs, soff);
                su_[p][u] = buf_load4(rus, soff);
            }
        }
        stage_x_tile<XT>(smem, a.x, GH * CPGX);  // after the weight stream is issued
        __syncthreads();
        float accg[kK2Pairs], accu[kK2Pairs];
#pragma unroll
        for (int p = 0; p < kK2Pairs; ++p) accg[p] = accu[p] = 0.f;
#pragma unroll
        for (int u = 0; u < GA; ++u) {
            const int g = u * 64 + lane;
            if (g < GH) {
                XChunk<XT> xc[CPGX];
#pragma unroll
                for (int q = 0; q < CPGX; ++q) xc[q] = reinterpret_cast<const XChunk<XT> *>(smem)[XTile<XT>::slot(g, q)];
#pragma unroll
                for (int p = 0; p < kK2Pairs; ++p) {
                    const uint32_t so = static_cast<uint32_t>(ii[p] * GH);
                    accg[p] = fmaf(group_dot(wg_[p][u], xc), e8m0_to_f32(scale_byte(sg_[p][u], so, g)), accg[p]);
                    accu[p] = fmaf(group_dot(wu_[p][u], xc), e8m0_to_f32(scale_byte(su_[p][u], so, g)), accu[p]);
                }
            }
        }
#pragma unroll
        for (int p = 0; p < kK2Pairs; ++p) {
            const float g = wave_sum_to_lane63(accg[p]);
            const float u = wave_sum_to_lane63(accu[p]);
            if (lane == 63 && vv[p])
                a.ws.act[static_cast<int64_t>(jj[p]) * a.I + ii[p]] = act_fn(g, u, a.act_kind, a.beta, a.lbeta);
        }
    } else {
        // shared down: bf16 [H, Is] rows against shared_act (fp32), 2 rows per wave
        uint4 *al = smem;
        const int n = ((blockIdx.x - a.k2_routed_blocks) * 4 + wave) * 2;
        const uint32_t row_bytes = static_cast<uint32_t>(a.Is) * 2u;
        const auto rr = make_rsrc(a.sh_down, static_cast<uint32_t>(a.H) * row_bytes);
        const __amdgpu_buffer_rsrc_t r[2] = {rr, rr};
        const uint32_t off[2] = {static_cast<uint32_t>(n) * row_bytes, static_cast<uint32_t>(n + 1) * row_bytes};
        const bool v[2] = {n < a.H, n + 1 < a.H};
        uint4 w[2][CHI];
        bf16_rows_load<CHI, 2>(r, off, a.Is, v, w);
        stage_plain<float>(al, a.ws.shared_act, a.Is);
        __syncthreads();
        float t[2];
        bf16_rows_dot<float, CHI, 2>(w, a.Is, al, t);
        if (lane == 63) {
            if (v[0]) a.ws.yshared[n] = t[0];
            if (v[1]) a.ws.yshared[n + 1] = t[1];
        }
    }
}

// ------------------------------------------------------------------ K3
// Blocks of 8 waves; each wave owns RPW output rows and needs the KT routed down rows of
// each (K = I, GB groups per lane).  Order of work per block:
//   1. the k experts' act vectors (L2-resident, 8 KB each) are loaded into registers and
//      the scale dwords are issued,
//   2. the whole weight stream (KT x RPW rows) is issued,
//   3. act goes to LDS (that wait covers only the loads of step 1),
//   4. experts are consumed in issue order, so compute overlaps the stream's tail.
constexpr int kK3Waves = 8;

template <int KT, int RPW, int GB>
__global__ __launch_bounds__(512) void layer_k3(LayerArgs a) {
    extern __shared__ uint4 smem[];
    __shared__ uint64_t tab_s[kMaxTopK][2];
    __shared__ float w_s[kMaxTopK];
    constexpr int NT = kK3Waves * 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int GI = a.I >> 5;
    const uint32_t rowB = static_cast<uint32_t>(a.I >> 1);
    if (static_cast<int>(threadIdx.x) < KT) {
        tab_s[threadIdx.x][0] = a.ws.sel_ptrs[threadIdx.x * 6 + 4];
        tab_s[threadIdx.x][1] = a.ws.sel_ptrs[threadIdx.x * 6 + 5];
        w_s[threadIdx.x] = a.ws.topk_w[threadIdx.x];
    }
    // 1. act chunks into registers (one fp32 tile of GI*8 chunks per expert slot)
    const int per = GI * 8;
    constexpr int AREG = KT * 64 * 8 / NT;  // chunks per thread at I <= 2048 per GB
    uint4 av[AREG * GB];
    {
        const auto ra = make_rsrc(a.ws.act, static_cast<uint32_t>(KT * per * 16));
#pragma unroll
        for (int b = 0; b < AREG * GB; ++b) {
            const int c = b * NT + threadIdx.x;
            av[b] = buf_load16(ra, c < KT * per ? static_cast<uint32_t>(c) * 16u : kOobOffset);
        }
    }
    __syncthreads();  // tab_s
    const int n0 = (blockIdx.x * kK3Waves + wave) * RPW;
    uint4 wd[KT][RPW][GB];
    uint32_t sd[KT][RPW][GB];
#pragma unroll
    for (int j = 0; j < KT; ++j) {
        const auto rds = make_rsrc(uniform_ptr(tab_s[j][1]), static_cast<uint32_t>(a.H * GI));
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int u = 0; u < GB; ++u) {
                const int n = n0 + r, g = u * 64 + lane;
                const bool ok = n < a.H && g < GI;
                sd[j][r][u] = buf_load4(rds, ok ? scale_dword_off(static_cast<uint32_t>(n * GI), g) : kOobOffset);
            }
    }
    // 2. the weight stream
#pragma unroll
    for (int j = 0; j < KT; ++j) {
        const auto rd = make_rsrc(uniform_ptr(tab_s[j][0]), static_cast<uint32_t>(a.H) * rowB);
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int u = 0; u < GB; ++u) {
                const int n = n0 + r, g = u * 64 + lane;
                const bool ok = n < a.H && g < GI;
                wd[j][r][u] = buf_load16(rd, ok ? static_cast<uint32_t>(n) * rowB + g * 16u : kOobOffset);
            }
    }
    // 3. act to LDS
#pragma unroll
    for (int b = 0; b < AREG * GB; ++b) {
        const int c = b * NT + threadIdx.x;
        if (c < KT * per) {
            const int j = c / per, cc = c % per;
            smem[j * per + XTile<float>::slot(cc >> 3, cc & 7)] = av[b];
        }
    }
    __syncthreads();
    // 4. consume in issue order
    float y[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) y[r] = 0.f;
#pragma unroll
    for (int j = 0; j < KT; ++j) {
        const uint4 *al = smem + j * per;
        float acc[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[r] = 0.f;
#pragma unroll
        for (int u = 0; u < GB; ++u) {
            const int g = u * 64 + lane;
            if (g < GI) {
                float4 ac[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) ac[q] = reinterpret_cast<const float4 *>(al)[XTile<float>::slot(g, q)];
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const int n = n0 + r;
                    acc[r] = fmaf(group_dot(wd[j][r][u], ac),
                                  e8m0_to_f32(scale_byte(sd[j][r][u], static_cast<uint32_t>(n * GI), g)), acc[r]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) y[r] = fmaf(w_s[j], wave_sum_to_lane63(acc[r]), y[r]);
    }
    if (lane == 63) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int n = n0 + r;
            if (n < a.H) {
                const float v = y[r] + (a.sh_down ? a.ws.yshared[n] : 0.f);
                if (a.out_bf16)
                    static_cast<uint16_t *>(a.out)[n] = f32_to_bf16(v);
                else
                    static_cast<float *>(a.out)[n] = v;
            }
        }
    }
}

// ------------------------------------------------------------------ host side
struct LayerWsLayout {
    size_t logits, scores, corrected, idx, w, shared_act, act, yshared, ptrs, total;
};

static size_t up256(size_t v) { return (v + 255) & ~size_t(255); }

static LayerWsLayout layer_ws_layout(int64_t H, int64_t I, int64_t Is, int64_t E, int64_t k) {
    LayerWsLayout L{};
    size_t o = 0;
    L.logits = o, o += up256(E * 4);
    L.scores = o, o += up256(E * 4);
    L.corrected = o, o += up256(E * 4);
    L.idx = o, o += up256(k * 4);
    L.w = o, o += up256(k * 4);
    L.shared_act = o, o += up256(std::max<int64_t>(Is, 1) * 4);
    L.act = o, o += up256(k * I * 4);
    L.yshared = o, o += up256(H * 4);
    L.ptrs = o, o += up256(k * 6 * 8);
    L.total = o;
    return L;
}

static int launch_route(const LayerArgs &a, hipStream_t st) {
    const int threads = static_cast<int>(std::max<int64_t>(64, cdiv(a.E, 64) * 64));
    layer_route<<<dim3(1), threads, 0, st>>>(a);
    return check_hip(hipGetLastError(), "moe layer route");
}

template <typename XT>
static int launch_layer(LayerArgs &a, hipStream_t st) {
    const int GH = a.H / 32, GI = a.I / 32;
    const int chh = cdiv(a.H / 8, 64);        // bf16 chunks per lane over H
    const int chi = cdiv(a.Is / 8, 64);       // over Is
    const int ga = GH <= 128 ? 2 : (GH <= 256 ? 4 : 0);
    const int gb = GI <= 64 ? 1 : (GI <= 128 ? 2 : 0);
    if (!ga || !gb || chh > 16 || (a.sh_down && chi > 8))
        return set_error(K3_ERR_SHAPE, "moe layer: H=%d I=%d Is=%d outside the kernels' range", a.H, a.I, a.Is);
    // K1
    a.k1_router_blocks = static_cast<int>(cdiv(a.E, 4));
    const int k1_blocks = a.k1_router_blocks + (a.sh_gate ? static_cast<int>(cdiv(a.Is, 4)) : 0);
    const size_t lds1 = static_cast<size_t>(a.H) * sizeof(XT);
#define K1(C) \
    if (chh <= C) { layer_k1<XT, C><<<dim3(k1_blocks), 256, lds1, st>>>(a); } else
    K1(4) K1(8) K1(12) K1(16) {}
#undef K1
    int rc = check_hip(hipGetLastError(), "moe layer K1");
    if (rc) return rc;
    rc = launch_route(a, st);
    if (rc) return rc;
    // K2
    a.k2_routed_blocks = static_cast<int>(cdiv(static_cast<int64_t>(a.k) * a.I, 4 * kK2Pairs));
    const int k2_blocks = a.k2_routed_blocks + (a.sh_down ? static_cast<int>(cdiv(a.H, 8)) : 0);
    const size_t lds2 = std::max<size_t>(static_cast<size_t>(GH) * XTile<XT>::kChunks * 16,
                                         static_cast<size_t>(a.Is) * 4);
#define K2(G_, C_) \
    if (ga == G_ && chi <= C_) { layer_k2<XT, G_, C_><<<dim3(k2_blocks), 256, lds2, st>>>(a); } else
    K2(2, 4) K2(2, 8) K2(4, 4) K2(4, 8) {}
#undef K2
    rc = check_hip(hipGetLastError(), "moe layer K2");
    if (rc) return rc;
    // K3: 4 rows per wave at I <= 2048, 2 rows per wave above (register budget)
    const int rpw = gb == 1 ? 4 : 2;
    const int k3_blocks = static_cast<int>(cdiv(a.H, kK3Waves * rpw));
    const size_t lds3 = static_cast<size_t>(a.k) * a.I * 4;
    const void *f3 = nullptr;
#define K3SEL(KT_, GB_, R_) \
    if (a.k == KT_ && gb == GB_) f3 = reinterpret_cast<const void *>(&layer_k3<KT_, R_, GB_>);
    K3SEL(1, 1, 4) K3SEL(2, 1, 4) K3SEL(4, 1, 4) K3SEL(6, 1, 4) K3SEL(8, 1, 4)
    K3SEL(1, 2, 2) K3SEL(2, 2, 2) K3SEL(4, 2, 2) K3SEL(8, 2, 2)
#undef K3SEL
    if (!f3) return set_error(K3_ERR_SHAPE, "moe layer: no combine kernel for top_k=%d, I=%d", a.k, a.I);
    if (lds3 + 1024 > 64 * 1024) {
        rc = check_hip(hipFuncSetAttribute(f3, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds3)),
                       "moe layer K3 LDS limit");
        if (rc) return rc;
    }
#define K3RUN(KT_, GB_, R_) \
    if (a.k == KT_ && gb == GB_) layer_k3<KT_, R_, GB_><<<dim3(k3_blocks), kK3Waves * 64, lds3, st>>>(a);
    K3RUN(1, 1, 4) K3RUN(2, 1, 4) K3RUN(4, 1, 4) K3RUN(6, 1, 4) K3RUN(8, 1, 4)
    K3RUN(1, 2, 2) K3RUN(2, 2, 2) K3RUN(4, 2, 2) K3RUN(8, 2, 2)
#undef K3RUN
    return check_hip(hipGetLastError(), "moe layer K3");
}

}  // namespace k3

using namespace k3;

static int route_only(LayerArgs &a, int x_bf16, hipStream_t st) {
    const int chh = static_cast<int>(cdiv(a.H / 8, 64));
    if (chh > 16) return set_error(K3_ERR_SHAPE, "moe route: H=%d too wide", a.H);
    a.k1_router_blocks = static_cast<int>(cdiv(a.E, 4));
    const size_t lds1 = static_cast<size_t>(a.H) * (x_bf16 ? 2 : 4);
#define K1(C) \
    if (chh <= C) { \
        if (x_bf16) layer_k1<uint16_t, C><<<dim3(a.k1_router_blocks), 256, lds1, st>>>(a); \
        else layer_k1<float, C><<<dim3(a.k1_router_blocks), 256, lds1, st>>>(a); \
    } else
    K1(4) K1(8) K1(12) K1(16) {}
#undef K1
    int rc = check_hip(hipGetLastError(), "moe route K1");
    if (rc) return rc;
    return launch_route(a, st);
}

extern "C" int64_t k3_moe_layer_workspace_size(int64_t H, int64_t I, int64_t shared_I, int64_t n_experts,
                                               int64_t top_k) {
    return static_cast<int64_t>(layer_ws_layout(H, I, shared_I, n_experts, top_k).total);
}

static int layer_impl(const void *x, int x_dtype, const void *router_w, const void *router_bias, int route_kind,
                      int renormalize, float scaling, const void *expert_table, const void *shared_gate,
                      const void *shared_up, const void *shared_down, void *out, int out_dtype, int64_t H, int64_t I,
                      int64_t shared_I, int64_t n_experts, int64_t top_k, int act_kind, float beta, float linear_beta,
                      void *workspace, int64_t workspace_bytes, void *stream, bool route_only_flag) {
    if (!x || !router_w || !workspace || (!route_only_flag && (!expert_table || !out)))
        return set_error(K3_ERR_NULL, "moe layer: null pointer");
    const bool has_shared = shared_gate || shared_up || shared_down;
    if (has_shared && !(shared_gate && shared_up && shared_down))
        return set_error(K3_ERR_NULL, "moe layer: shared expert needs gate, up and down");
    if (x_dtype != K3_F32 && x_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "moe layer: x_dtype");
    if (out_dtype != K3_F32 && out_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "moe layer: out_dtype");
    if (route_kind != K3_ROUTE_SOFTMAX && route_kind != K3_ROUTE_SIGMOID_BIAS)
        return set_error(K3_ERR_SHAPE, "moe layer: route_kind");
    if (act_kind != K3_ACT_SILU && act_kind != K3_ACT_SITU) return set_error(K3_ERR_SHAPE, "moe layer: act_kind");
    if (H <= 0 || I <= 0 || H % 128 || I % 128 || (has_shared && (shared_I <= 0 || shared_I % 128)))
        return set_error(K3_ERR_SHAPE, "moe layer: H, I and shared_I must be positive multiples of 128");
    if (n_experts <= 0 || n_experts > kMaxExperts || top_k <= 0 || top_k > kMaxTopK || top_k > n_experts)
        return set_error(K3_ERR_SHAPE, "moe layer: n_experts must be in 1..%d and top_k in 1..min(%d, n_experts)",
                         kMaxExperts, kMaxTopK);
    if (top_k * I * 4 > 160 * 1024)
        return set_error(K3_ERR_SHAPE, "moe layer: top_k * I = %lld exceeds the combine kernel's LDS",
                         (long long)(top_k * I));
    const LayerWsLayout L = layer_ws_layout(H, I, has_shared ? shared_I : 0, n_experts, top_k);
    if (workspace_bytes < static_cast<int64_t>(L.total))
        return set_error(K3_ERR_WORKSPACE, "moe layer: workspace %lld < %zu bytes", (long long)workspace_bytes, L.total);
    if (!aligned16(x) || !aligned16(router_w) || !aligned16(workspace) ||
        (has_shared && (!aligned16(shared_gate) || !aligned16(shared_up) || !aligned16(shared_down))))
        return set_error(K3_ERR_ALIGN, "moe layer: x, weights and workspace must be 16-byte aligned");
    if (n_experts * H * 2 >= (1ll << 31) || H * I / 2 >= (1ll << 31) || (has_shared && H * shared_I * 2 >= (1ll << 31)))
        return set_error(K3_ERR_SHAPE, "moe layer: a weight matrix exceeds 2 GiB");
    char *w = static_cast<char *>(workspace);
    LayerArgs a{};
    a.x = x;
    a.router_w = static_cast<const uint16_t *>(router_w);
    a.router_bias = static_cast<const float *>(router_bias);
    a.table = static_cast<const uint64_t *>(expert_table);
    a.sh_gate = static_cast<const uint16_t *>(shared_gate);
    a.sh_up = static_cast<const uint16_t *>(shared_up);
    a.sh_down = static_cast<const uint16_t *>(shared_down);
    a.out = out;
    a.ws.logits = reinterpret_cast<float *>(w + L.logits);
    a.ws.scores = reinterpret_cast<float *>(w + L.scores);
    a.ws.corrected = reinterpret_cast<float *>(w + L.corrected);
    a.ws.topk_idx = reinterpret_cast<int32_t *>(w + L.idx);
    a.ws.topk_w = reinterpret_cast<float *>(w + L.w);
    a.ws.shared_act = reinterpret_cast<float *>(w + L.shared_act);
    a.ws.act = reinterpret_cast<float *>(w + L.act);
    a.ws.yshared = reinterpret_cast<float *>(w + L.yshared);
    a.ws.sel_ptrs = reinterpret_cast<uint64_t *>(w + L.ptrs);
    a.H = static_cast<int>(H);
    a.I = static_cast<int>(I);
    a.Is = has_shared ? static_cast<int>(shared_I) : 0;
    a.E = static_cast<int>(n_experts);
    a.k = static_cast<int>(top_k);
    a.route_kind = route_kind;
    a.renorm = renormalize;
    a.scaling = scaling;
    a.act_kind = act_kind;
    a.beta = beta;
    a.lbeta = linear_beta;
    a.out_bf16 = out_dtype == K3_BF16;
    auto st = static_cast<hipStream_t>(stream);
    if (route_only_flag) return route_only(a, x_dtype == K3_BF16, st);
    return x_dtype == K3_BF16 ? launch_layer<uint16_t>(a, st) : launch_layer<float>(a, st);
}

extern "C" int k3_moe_layer_decode(const void *x, int x_dtype, const void *router_w, const void *router_bias,
                                   int route_kind, int renormalize, float scaling, const void *expert_table,
                                   const void *shared_gate, const void *shared_up, const void *shared_down,
                                   void *out, int out_dtype, int64_t H, int64_t I, int64_t shared_I,
                                   int64_t n_experts, int64_t top_k, int act_kind, float beta, float linear_beta,
                                   void *workspace, int64_t workspace_bytes, void *stream) {
    return layer_impl(x, x_dtype, router_w, router_bias, route_kind, renormalize, scaling, expert_table, shared_gate,
                      shared_up, shared_down, out, out_dtype, H, I, shared_I, n_experts, top_k, act_kind, beta,
                      linear_beta, workspace, workspace_bytes, stream, false);
}

extern "C" int k3_moe_route(const void *x, int x_dtype, const void *router_w, const void *router_bias, int route_kind,
                            int renormalize, float scaling, int64_t H, int64_t n_experts, int64_t top_k,
                            void *workspace, int64_t workspace_bytes, void *stream) {
    return layer_impl(x, x_dtype, router_w, router_bias, route_kind, renormalize, scaling, nullptr, nullptr, nullptr,
                      nullptr, nullptr, K3_F32, H, 128, 0, n_experts, top_k, K3_ACT_SILU, 1.f, 0.f, workspace,
                      workspace_bytes, stream, true);
}

extern "C" int k3_moe_layer_workspace_offsets(int64_t H, int64_t I, int64_t shared_I, int64_t n_experts,
                                              int64_t top_k, int64_t *offsets) {
    if (!offsets) return set_error(K3_ERR_NULL, "moe layer offsets: null pointer");
    const LayerWsLayout L = layer_ws_layout(H, I, shared_I, n_experts, top_k);
    const size_t v[8] = {L.logits, L.scores, L.corrected, L.idx, L.w, L.shared_act, L.act, L.yshared};
    for (int i = 0; i < 8; ++i) offsets[i] = static_cast<int64_t>(v[i]);
    return K3_OK;
}
