// Grouped routed-expert FFN for many tokens (prefill): every routed (token, slot) pair is
// grouped by expert, and each expert runs as a GEMM with M = its token count, so each
// expert's MXFP4 weights stream from HBM once per 32-token tile group instead of once per
// token.
//
// Reference: LatentMoE.__call__ (air_llm/models/kimi_k3/moe.py:110-132; k3ref
// k3ref/layers.py:241-261): for each distinct routed expert, gather its tokens, run
// expert_forward, scale by the gate weight and add into y.  The reference loops over
// experts on the host; here:
//
//   count   block e counts the pairs routed to expert e                      -> counts[E]
//   plan    one block: exclusive scan of the counts (segment bases) and the list of
//           32-token tiles (expert, first row) of every non-empty expert
//   place   block e writes its pairs, in (token, slot) order, into perm[base_e ...]
//   gateup  block (tile, 128 intermediate rows): act = f(x W_gate^T, x W_up^T) for the
//           tile's tokens; bf16 MFMA (v_mfma_f32_16x16x32_bf16) on x (bf16) and the MXFP4
//           weights decoded in registers with their E8M0 scale folded in
//           (v_cvt_scalef32_pk_bf16_fp4: E2M1 x 2^e is exact in bf16); act is stored as a
//           bf16 hi/lo pair so the next product keeps fp32-class precision
//   down    block (tile, 256 output rows): y_pair = act W_down^T (MFMAs on act_hi and
//           act_lo) -> fp32 rows per (token, slot) pair
//   combine y[t] = sum_slot w[t, slot] * y_pair[t, slot], slots in order
//
// Deterministic: no atomics, fixed summation orders everywhere.
#include <algorithm>

#include "k3_common.h"
#include "moe_common.h"

namespace k3 {
namespace {

constexpr int kMt = 32;           // tokens per tile (two MFMA row tiles)
constexpr int kKs = 64;           // K per pipeline step (two MFMA k-steps)
constexpr int kNg = 256;          // weight rows per block (gate/up: 128 + 128)
constexpr int kThreads = 512;     // 8 waves: wave w owns weight rows [32 w, 32 w + 32)
constexpr int kARow = kKs + 8;    // padded bf16 A row in LDS (144 B)
constexpr int kBRow = 9;          // padded B row in LDS: 32 packed bytes + 4 pad, in dwords

typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct GroupArgs {
    const int32_t *idx;    // [P] expert id of pair p = t * k + slot
    int P, E;
    int32_t *counts;       // [E]
    int32_t *base;         // [E]
    int32_t *perm;         // [P]: pairs grouped by expert
    int32_t *tile_e;       // [max_tiles]
    int32_t *tile_m0;      // [max_tiles]
    int32_t *n_tiles;      // [1]
    int max_tiles;
};

// Stable compaction of the pairs equal to `e` (wave ballots, block prefix over 8 waves).
// Called by every thread of a 256-thread block; returns the block's total.
template <bool WRITE>
__device__ int scan_expert(const GroupArgs &g, int e, int32_t *out) {
    __shared__ int wcnt[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int total = 0;
    for (int p0 = 0; p0 < g.P; p0 += 256) {
        const int p = p0 + tid;
        const bool hit = p < g.P && g.idx[p] == e;
        const uint64_t m = __ballot(hit);
        if (lane == 0) wcnt[wave] = __popcll(m);
        __syncthreads();
        int before = total;
        for (int w = 0; w < wave; ++w) before += wcnt[w];
        if (WRITE && hit) out[before + __popcll(m & ((1ull << lane) - 1ull))] = p;
        total += wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
        __syncthreads();
    }
    return total;
}

__global__ __launch_bounds__(256) void group_count_kernel(GroupArgs g) {
    const int n = scan_expert<false>(g, blockIdx.x, nullptr);
    if (threadIdx.x == 0) g.counts[blockIdx.x] = n;
}

__global__ __launch_bounds__(256) void group_place_kernel(GroupArgs g) {
    scan_expert<true>(g, blockIdx.x, g.perm + g.base[blockIdx.x]);
}

// One block of 1024 threads: segment bases and the tile list (E <= 1024).
__global__ __launch_bounds__(1024) void group_plan_kernel(GroupArgs g) {
    __shared__ int sc[1024], st[1024];
    const int e = threadIdx.x;
    const int c = e < g.E ? g.counts[e] : 0;
    sc[e] = c;
    st[e] = (c + kMt - 1) / kMt;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {  // inclusive Hillis-Steele scans
        const int a = e >= off ? sc[e - off] : 0, b = e >= off ? st[e - off] : 0;
        __syncthreads();
        sc[e] += a;
        st[e] += b;
        __syncthreads();
    }
    if (e < g.E) {
        g.base[e] = sc[e] - c;
        const int t0 = st[e] - (c + kMt - 1) / kMt;
        for (int j = 0; j * kMt < c; ++j) {
            if (t0 + j < g.max_tiles) {
                g.tile_e[t0 + j] = e;
                g.tile_m0[t0 + j] = j * kMt;
            }
        }
    }
    if (e == 1023) *g.n_tiles = min(st[1023], g.max_tiles);
}

// ------------------------------------------------------------------ grouped GEMMs
struct GemmArgs {
    const uint16_t *x;       // gate/up: [T, K] bf16 token rows
    const uint16_t *a_hi;    // down: act hi [P, K] bf16, rows in grouped order
    const uint16_t *a_lo;    // down: act lo
    const uint64_t *table;   // [E][6] expert pointers
    const int32_t *counts, *base, *perm, *tile_e, *tile_m0, *n_tiles;
    uint16_t *act_hi, *act_lo;  // gate/up output [P, I]
    float *ypair;            // down output [P, H]: row = pair id
    int K, N, top_k;         // K: reduction length; N: weight rows of one projection
    int nt_per_tile;         // weight-row blocks per tile
    int max_tiles;
    int act_kind;
    float beta, lbeta;
};

__device__ __forceinline__ f32x4_t mfma_bf16(bf16x8 a, bf16x8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 8 packed E2M1 codes (one dword) -> 8 bf16 scaled by 2^(e-127), exact for normal results
__device__ __forceinline__ bf16x8 decode8(uint32_t w, float s) {
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 0);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 1);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 2);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, s, 3);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// DOWN == false: gate/up + activation (weights rows 0..127 gate, 128..255 up of the same
// 128 intermediate indices).  DOWN == true: 256 output rows of W_down, A = act hi/lo.
template <bool DOWN>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(GemmArgs a) {
    constexpr int AH = DOWN ? 2 : 1;  // A planes (hi, lo)
    __shared__ __align__(16) uint16_t a_s[2][AH][kMt * kARow];
    __shared__ __align__(16) uint32_t b_s[2][kNg * kBRow];
    __shared__ uint16_t sc_s[2][kNg];
    __shared__ float g_s[DOWN ? 1 : kMt * 129];  // gate results for the epilogue

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = static_cast<int>(gridDim.x);
    const int w = (nb & 7) == 0 ? (blockIdx.x & 7) * (nb >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const int tile = w % a.max_tiles, nt = w / a.max_tiles;
    if (tile >= *a.n_tiles) return;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    const int cnt = a.counts[e];
    const int rows = min(kMt, cnt - m0);
    const int pos0 = a.base[e] + m0;  // grouped row of the tile's first token
    const uint64_t *ptr = a.table + static_cast<int64_t>(e) * 6;
    const int KG = a.K >> 5;          // scale groups per weight row
    const uint32_t rowb = static_cast<uint32_t>(a.K >> 1);

    // ---- per-thread load assignments
    // A: row r = c >> 3, 16-byte chunk c & 7 of the step's 128 bytes (threads 0..255 per plane)
    const int ac = tid & 255, ar = ac >> 3, ach = ac & 7, aplane = DOWN ? (tid >> 8) : 0;
    const bool a_thread = DOWN || tid < 256;
    const uint16_t *arow = nullptr;
    if (a_thread && ar < rows) {
        if (DOWN) {
            arow = (aplane ? a.a_lo : a.a_hi) + static_cast<int64_t>(pos0 + ar) * a.K;
        } else {
            const int pair = a.perm[pos0 + ar];
            arow = a.x + static_cast<int64_t>(pair / a.top_k) * a.K;
        }
    }
    // B: weight row br = tid >> 1 (of 256), 16-byte half bh of the step's 32 bytes
    const int br = tid >> 1, bh = tid & 1;
    int wrow;
    const uint8_t *bp, *bs;
    if (DOWN) {
        wrow = nt * kNg + br;
        bp = reinterpret_cast<const uint8_t *>(ptr[4]);
        bs = reinterpret_cast<const uint8_t *>(ptr[5]);
    } else {
        wrow = nt * (kNg / 2) + (br & 127);
        bp = reinterpret_cast<const uint8_t *>(ptr[br < 128 ? 0 : 2]);
        bs = reinterpret_cast<const uint8_t *>(ptr[br < 128 ? 1 : 3]);
    }
    const bool b_ok = wrow < a.N;
    const uint8_t *brow = bp + static_cast<int64_t>(b_ok ? wrow : 0) * rowb + bh * 16;
    const uint8_t *srow = bs + static_cast<int64_t>(b_ok ? wrow : 0) * KG;

    // three pipeline steps of operands in flight per thread: one step's MFMA work is far
    // shorter than a memory round trip
    constexpr int kDepth = 3;
    uint4 ra[kDepth], rb[kDepth];
    uint16_t rs[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
        ra[d] = make_uint4(0u, 0u, 0u, 0u);
        rb[d] = make_uint4(0u, 0u, 0u, 0u);
        rs[d] = 0;
    }
    auto load = [&](int ks, uint4 &va, uint4 &vb, uint16_t &vs) {
        const int k0 = ks * kKs;
        if (arow) va = *reinterpret_cast<const uint4 *>(arow + k0 + ach * 8);
        if (b_ok) {
            vb = *reinterpret_cast<const uint4 *>(brow + (k0 >> 1));
            if (bh == 0) vs = *reinterpret_cast<const uint16_t *>(srow + (k0 >> 5));
        }
    };
    auto store = [&](int buf, const uint4 &va, const uint4 &vb, uint16_t vs) {
        if (a_thread) *reinterpret_cast<uint4 *>(&a_s[buf][aplane][ar * kARow + ach * 8]) = va;
        uint32_t *bd = &b_s[buf][br * kBRow + bh * 4];
        bd[0] = vb.x;
        bd[1] = vb.y;
        bd[2] = vb.z;
        bd[3] = vb.w;
        if (bh == 0) sc_s[buf][br] = vs;
    };

    f32x4_t acc[2][2];  // [token tile][weight-row tile]
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int r16 = lane & 15, q4 = lane >> 4;
    const int nsteps = a.K / kKs;
    auto step = [&](int ks, int d) {
        const int buf = ks & 1;
        store(buf, ra[d], rb[d], rs[d]);
        __syncthreads();
        if (ks + kDepth < nsteps) load(ks + kDepth, ra[d], rb[d], rs[d]);
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            bf16x8 bop[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int row = wave * 32 + j * 16 + r16;
                const uint32_t pk = b_s[buf][row * kBRow + sub * 4 + q4];
                const uint32_t sb = (sc_s[buf][row] >> (8 * sub)) & 0xffu;
                bop[j] = decode8(pk, e8m0_to_f32(sb));
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
#pragma unroll
                for (int pl = 0; pl < AH; ++pl) {
                    const bf16x8 aop =
                        *reinterpret_cast<const bf16x8 *>(&a_s[buf][pl][(i * 16 + r16) * kARow + sub * 32 + q4 * 8]);
#pragma unroll
                    for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16(aop, bop[j], acc[i][j]);
                }
            }
        }
    };
#pragma unroll
    for (int d = 0; d < kDepth; ++d)
        if (d < nsteps) load(d, ra[d], rb[d], rs[d]);
    for (int ks = 0; ks < nsteps; ks += kDepth) {
        step(ks, 0);
        if (ks + 1 < nsteps) step(ks + 1, 1);
        if (ks + 2 < nsteps) step(ks + 2, 2);
    }

    // ---- epilogues.  C layout: lane holds tokens 16 i + 4 q4 + v (v < 4), weight row 16 j + r16
    if constexpr (DOWN) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int r = i * 16 + q4 * 4 + v;
                if (r < rows) {
                    const int pair = a.perm[pos0 + r];
                    float *yrow = a.ypair + static_cast<int64_t>(pair) * a.N + nt * kNg + wave * 32;
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        if (nt * kNg + wave * 32 + j * 16 + r16 < a.N) yrow[j * 16 + r16] = acc[i][j][v];
                }
            }
    } else {
        __syncthreads();
        if (wave < 4) {  // gate rows: publish to LDS
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        g_s[(i * 16 + q4 * 4 + v) * 129 + wave * 32 + j * 16 + r16] = acc[i][j][v];
        }
        __syncthreads();
        if (wave >= 4) {  // up rows: combine with the gate of the same intermediate index
            const int wl = wave - 4;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int r = i * 16 + q4 * 4 + v;
                    if (r >= rows) continue;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int il = wl * 32 + j * 16 + r16;
                        const int ii = nt * (kNg / 2) + il;
                        if (ii < a.N) {
                            const float act = act_fn(g_s[r * 129 + il], acc[i][j][v], a.act_kind, a.beta, a.lbeta);
                            const uint16_t hi = f32_to_bf16(act);
                            const int64_t o = static_cast<int64_t>(pos0 + r) * a.N + ii;
                            a.act_hi[o] = hi;
                            a.act_lo[o] = f32_to_bf16(act - bf16_to_f32(hi));
                        }
                    }
                }
        }
    }
}

// ------------------------------------------------------------------ combine
struct CombineArgs {
    const float *ypair;   // [T * k, H]
    const float *w;       // [T, k]
    void *out;            // [T, H]
    int T, H, k;
    int out_bf16;
};

// grid: (T, cdiv(H, 1024)); thread: 4 consecutive columns
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
    const int t = blockIdx.x;
    const int c = (blockIdx.y * 256 + threadIdx.x) * 4;
    if (c >= a.H) return;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < a.k; ++j) {
        const float wj = a.w[t * a.k + j];
        const float4 v = *reinterpret_cast<const float4 *>(a.ypair + static_cast<int64_t>(t * a.k + j) * a.H + c);
        s.x = fmaf(wj, v.x, s.x);
        s.y = fmaf(wj, v.y, s.y);
        s.z = fmaf(wj, v.z, s.z);
        s.w = fmaf(wj, v.w, s.w);
    }
    const int64_t o = static_cast<int64_t>(t) * a.H + c;
    if (a.out_bf16) {
        uint16_t *p = static_cast<uint16_t *>(a.out) + o;
        p[0] = f32_to_bf16(s.x);
        p[1] = f32_to_bf16(s.y);
        p[2] = f32_to_bf16(s.z);
        p[3] = f32_to_bf16(s.w);
    } else {
        *reinterpret_cast<float4 *>(static_cast<float *>(a.out) + o) = s;
    }
}

// ------------------------------------------------------------------ host side
struct GroupedWs {
    size_t counts, base, perm, tile_e, tile_m0, n_tiles, act_hi, act_lo, ypair, total;
    int max_tiles;
};

GroupedWs grouped_ws_layout(int64_t T, int64_t k, int64_t E, int64_t H, int64_t I) {
    GroupedWs L{};
    auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
    const int64_t P = T * k;
    L.max_tiles = static_cast<int>(cdiv(P, kMt) + E);
    size_t o = 0;
    L.counts = o, o += up(E * 4);
    L.base = o, o += up(E * 4);
    L.perm = o, o += up(P * 4);
    L.tile_e = o, o += up(static_cast<size_t>(L.max_tiles) * 4);
    L.tile_m0 = o, o += up(static_cast<size_t>(L.max_tiles) * 4);
    L.n_tiles = o, o += up(4);
    L.act_hi = o, o += up(static_cast<size_t>(P) * I * 2);
    L.act_lo = o, o += up(static_cast<size_t>(P) * I * 2);
    L.ypair = o, o += up(static_cast<size_t>(P) * H * 4);
    L.total = o;
    return L;
}

}  // namespace
}  // namespace k3

using namespace k3;

extern "C" int64_t k3_moe_grouped_workspace_size(int64_t T, int64_t top_k, int64_t n_experts, int64_t H, int64_t I) {
    if (T <= 0 || top_k <= 0 || n_experts <= 0 || H <= 0 || I <= 0) return 0;
    return static_cast<int64_t>(grouped_ws_layout(T, top_k, n_experts, H, I).total);
}

extern "C" int k3_moe_grouped_ffn(const void *x, int x_dtype, const int32_t *expert_idx, const float *expert_w,
                                  const void *expert_table, void *out, int out_dtype, int64_t T, int64_t H, int64_t I,
                                  int64_t n_experts, int64_t top_k, int act_kind, float beta, float linear_beta,
                                  void *workspace, int64_t workspace_bytes, void *stream) {
    if (!x || !expert_idx || !expert_w || !expert_table || !out || !workspace)
        return set_error(K3_ERR_NULL, "moe grouped: null pointer");
    if (x_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "moe grouped: x must be bf16 (x_dtype %d)", x_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "moe grouped: out_dtype");
    if (act_kind != K3_ACT_SILU && act_kind != K3_ACT_SITU) return set_error(K3_ERR_SHAPE, "moe grouped: act_kind");
    if (T <= 0 || top_k <= 0 || top_k > 64 || n_experts <= 0 || n_experts > 1024)
        return set_error(K3_ERR_SHAPE, "moe grouped: T >= 1, 1 <= top_k <= 64, 1 <= n_experts <= 1024 required");
    if (H <= 0 || I <= 0 || H % kKs || I % kKs || H % 4)
        return set_error(K3_ERR_SHAPE, "moe grouped: H=%lld and I=%lld must be positive multiples of %d",
                         (long long)H, (long long)I, kKs);
    if (T * top_k >= (1ll << 30) || H * I / 2 >= (1ll << 31))
        return set_error(K3_ERR_SHAPE, "moe grouped: problem too large");
    const GroupedWs L = grouped_ws_layout(T, top_k, n_experts, H, I);
    if (workspace_bytes < static_cast<int64_t>(L.total))
        return set_error(K3_ERR_WORKSPACE, "moe grouped: workspace %lld < %zu bytes", (long long)workspace_bytes,
                         L.total);
    if (!aligned16(x) || !aligned16(workspace) || !aligned16(out))
        return set_error(K3_ERR_ALIGN, "moe grouped: x, out and workspace must be 16-byte aligned");
    auto st = static_cast<hipStream_t>(stream);
    char *ws = static_cast<char *>(workspace);
    const int P = static_cast<int>(T * top_k);

    GroupArgs g{};
    g.idx = expert_idx;
    g.P = P;
    g.E = static_cast<int>(n_experts);
    g.counts = reinterpret_cast<int32_t *>(ws + L.counts);
    g.base = reinterpret_cast<int32_t *>(ws + L.base);
    g.perm = reinterpret_cast<int32_t *>(ws + L.perm);
    g.tile_e = reinterpret_cast<int32_t *>(ws + L.tile_e);
    g.tile_m0 = reinterpret_cast<int32_t *>(ws + L.tile_m0);
    g.n_tiles = reinterpret_cast<int32_t *>(ws + L.n_tiles);
    g.max_tiles = L.max_tiles;
    group_count_kernel<<<dim3(g.E), 256, 0, st>>>(g);
    group_plan_kernel<<<dim3(1), 1024, 0, st>>>(g);
    group_place_kernel<<<dim3(g.E), 256, 0, st>>>(g);
    int rc = check_hip(hipGetLastError(), "moe grouped: grouping launches");
    if (rc) return rc;

    GemmArgs ga{};
    ga.x = static_cast<const uint16_t *>(x);
    ga.table = static_cast<const uint64_t *>(expert_table);
    ga.counts = g.counts;
    ga.base = g.base;
    ga.perm = g.perm;
    ga.tile_e = g.tile_e;
    ga.tile_m0 = g.tile_m0;
    ga.n_tiles = g.n_tiles;
    ga.act_hi = reinterpret_cast<uint16_t *>(ws + L.act_hi);
    ga.act_lo = reinterpret_cast<uint16_t *>(ws + L.act_lo);
    ga.ypair = reinterpret_cast<float *>(ws + L.ypair);
    ga.top_k = static_cast<int>(top_k);
    ga.max_tiles = L.max_tiles;
    ga.act_kind = act_kind;
    ga.beta = beta;
    ga.lbeta = linear_beta;
    // gate/up: K = H, weight rows N = I, 128 intermediate indices per block
    ga.K = static_cast<int>(H);
    ga.N = static_cast<int>(I);
    ga.nt_per_tile = static_cast<int>(cdiv(I, kNg / 2));
    grouped_gemm_kernel<false><<<dim3(static_cast<unsigned>(L.max_tiles * ga.nt_per_tile)), kThreads, 0, st>>>(ga);
    rc = check_hip(hipGetLastError(), "moe grouped: gate/up launch");
    if (rc) return rc;
    // down: K = I, weight rows N = H, 256 output rows per block
    ga.a_hi = ga.act_hi;
    ga.a_lo = ga.act_lo;
    ga.K = static_cast<int>(I);
    ga.N = static_cast<int>(H);
    ga.nt_per_tile = static_cast<int>(cdiv(H, kNg));
    grouped_gemm_kernel<true><<<dim3(static_cast<unsigned>(L.max_tiles * ga.nt_per_tile)), kThreads, 0, st>>>(ga);
    rc = check_hip(hipGetLastError(), "moe grouped: down launch");
    if (rc) return rc;

    CombineArgs ca{ga.ypair, expert_w, out, static_cast<int>(T), static_cast<int>(H), static_cast<int>(top_k),
                   out_dtype == K3_BF16};
    combine_kernel<<<dim3(static_cast<unsigned>(T), static_cast<unsigned>(cdiv(H, 1024))), 256, 0, st>>>(ca);
    return check_hip(hipGetLastError(), "moe grouped: combine launch");
}
