// Routed experts for a few decode tokens (up to 8) in one pass: every expert any of the
// tokens selects is read from HBM once, against all the tokens routed to it.
//
// Reference: the dispatch loop of LatentMoE.__call__ (air_llm/models/kimi_k3/moe.py:119-127;
// k3ref/layers.py:241-261): for each distinct routed expert e, in ascending id, gather the
// tokens whose top-k holds e (h[ti]), run expert_forward on them together (the Metal kernel
// takes M tokens per launch, grid (N, M, 1), mxfp4_matvec.py:89-95), scale each token's
// output by its gate weight for e and add it into y.  A token is gathered once per expert,
// with the weight of its first slot holding e (list.index, moe.py:121-122).  Here, four
// stream-ordered launches and no host synchronisation:
//
//   U   one block: the union of the routed experts (distinct valid ids, ascending), each
//       union slot's (token, slot) pairs -- one per token, the token's first slot holding
//       the expert -- in token order, the slots' six weight pointers, a live flag per pair.
//   G   block (union slot u, 16 or 8 intermediate rows): each wave holds four or two (gate
//       row, up row) pairs of u's expert in registers and reduces them against every token of u, whose
//       rows are staged in LDS (up to tb_x tokens at a time, in the swizzled group order of
//       the batch-1 kernels) -> act[pair][i] = f(gate, up) in fp32.
//   D   block (union slot u, 4 * RW output rows): the rows of u's down projection in
//       registers, reduced against the act vector of each of u's pairs (staged in LDS, up to
//       tb_act at a time, chunk-major as the layer's down launch stages one); the row totals
//       per pair go to the workspace.
//   C   one thread per output value:
//       y[t] = yadd[t] + sum over the token's live slots j, in slot order, of w[t, j] * down_{t, j}
//       (yadd: the shared expert's output of the whole-layer entry point, or nothing).  A
//       launch of its own (the kernel boundary orders D's stores before its loads): combining
//       in D's last block per row range cost every D block a wait for its stores and an
//       arrival counter (without them K3's four-token D 94 -> 79 us, the 384-expert layer's
//       62 -> 51 us, for a 4.7 us combine launch).
//
// The whole layer for T tokens (k3_moe_layer_decode_multi) adds the dense bf16 parts on R, a
// row kernel for T tokens (4 waves, or 8 for fp32 inputs of 32-64 KB; one row or one
// (gate, up) row pair per wave, the T input rows staged in LDS once per block; wider fp32
// inputs take a persistent form that stages them once per CU): the router logits with the
// shared gate/up rows in one launch, the batched top-k (k3_moe_topk), U, G, D with the
// shared down rows as extra blocks of its launch, and C; with a side stream (the default) the
// shared expert's gate/up and down rows run there instead, beside R, the top-k, U, G and D.
// The latent layer (k3_moe_latent_layer_decode_multi) does the same.
//
// Every launch issues its weight rows before it waits on anything else, and loads what it
// stages in batches (every load of a batch issued before the first store), so a block's
// staging overlaps its weight stream instead of following it.
//
// Every selected expert's gate, up and down bytes are read once per call, whatever the
// number of tokens routed to it.  Deterministic: no float atomics, fixed orders.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <type_traits>

#include "moe_common.h"
#include "mxfp4_dot.h"

namespace k3 {
namespace {

constexpr int kMaxTokens = 8;
constexpr int kMaxTopK = 16;
constexpr int kMaxPairs = kMaxTokens * kMaxTopK;  // 128
constexpr int kMaxExperts = 1024;
// G: (gate, up) row pairs per wave: four for rows of up to 4096 values (K3's latent width:
// 134.7 -> 131.9 us per four-token step), two for wider rows (the 384-expert layer's 7168:
// four pairs measured 87.4 -> 90.2 us)
constexpr int g_pairs_per_wave(int GA) { return GA <= 2 ? 4 : 2; }
// LDS bytes per block for the staged token batches: small, so that LDS does not cap the
// blocks per CU below what the registers allow (the launches are bandwidth-bound)
constexpr int kLdsBudgetG = 16384;
constexpr int kLdsBudgetD = 40960;

struct MultiArgs {
    const void *x;           // [T, Hr] rows, bf16 or fp32
    const int32_t *idx;      // [T, k]
    const float *wts;        // [T, k]
    const uint64_t *table;   // [E][6] gate p/s, up p/s, down p/s
    void *out;               // [T, Hr]
    int T, Hr, I, E, k, P;
    int act_kind;
    float beta, lbeta;
    int out_bf16;
    int tb_x, tb_act;        // tokens per staged batch in G and D
    // workspace records
    int32_t *nu;             // [1] union size
    int32_t *u_count;        // [P] pairs of union slot u
    int32_t *u_pairs;        // [P][T] pair ids t * k + j of slot u, tokens ascending
    int32_t *live;           // [P] 1: pair contributes (valid id, the token's first slot holding it)
    uint64_t *u_ptrs;        // [P][6] weight pointers of slot u's expert
    float *act;              // [P][I] act of each live pair
    float *yrow;             // [P][Hr] down totals of each live pair
    const float *yadd;       // [T][Hr] added to each combined row (the shared expert) or null
};

// ------------------------------------------------------------------ U: the union
__global__ __launch_bounds__(256) void multi_union_kernel(MultiArgs a) {
    __shared__ int id_s[kMaxPairs];
    __shared__ int ex_s[kMaxPairs];
    __shared__ int first_s[kMaxPairs];
    __shared__ int nu_s;
    const int p = threadIdx.x;
    if (p == 0) nu_s = 0;
    const int v = p < a.P ? a.idx[p] : -1;  // every id loaded once, side by side
    if (p < kMaxPairs) id_s[p] = v;
    __syncthreads();
    int e = -1;
    if (p < a.P) {
        e = (v >= 0 && v < a.E) ? v : -1;
        const int t = p / a.k, j = p % a.k;
        int dup = 0;  // an earlier slot of the token holds it
#pragma unroll 8
        for (int jj = 0; jj < j; ++jj) dup |= id_s[t * a.k + jj] == v;
        if (dup) e = -1;
    }
    if (p < kMaxPairs) ex_s[p] = e;
    __syncthreads();
    // Scans over the pairs without branches, unrolled, so the LDS reads of a scan are in
    // flight together (a branch per element made every read wait for the one before).
    int pos = 0, cnt = 0;  // pairs of e before p; pairs of e
#pragma unroll 8
    for (int q = 0; q < a.P; ++q) {
        const int m = ex_s[q] == e;
        pos += m & (q < p);
        cnt += m;
    }
    const bool fst = e >= 0 && pos == 0;
    if (p < kMaxPairs) first_s[p] = fst;
    __syncthreads();
    if (e >= 0) {
        int slot = 0;  // distinct experts below e
#pragma unroll 8
        for (int q = 0; q < a.P; ++q) slot += first_s[q] & (ex_s[q] < e);
        a.u_pairs[slot * a.T + pos] = p;
        if (fst) {
            a.u_count[slot] = cnt;
#pragma unroll
            for (int c = 0; c < 6; ++c) a.u_ptrs[slot * 6 + c] = a.table[static_cast<int64_t>(e) * 6 + c];
            atomicAdd(&nu_s, 1);
        }
    }
    if (p < a.P) a.live[p] = e >= 0;
    __syncthreads();
    if (p == 0) *a.nu = nu_s;
}

// ------------------------------------------------------------------ G: gate/up + act
// GA: MXFP4 groups per lane over Hr (Hr <= 2048 * GA).
template <typename XT, int GA>
__global__ __launch_bounds__(256) void multi_gateup_kernel(MultiArgs a) {
    constexpr int kPairsPerWave = g_pairs_per_wave(GA);
    constexpr int kGRows = 4 * kPairsPerWave;  // intermediate rows per block
    extern __shared__ uint4 smem[];  // [tb_x][Hr / 8 (bf16) or Hr / 4 (fp32) chunks], swizzled
    __shared__ uint32_t tok_s[kMaxTokens];  // byte offsets of the slot's token rows in x
    __shared__ int pair_s[kMaxTokens];      // the slot's pair ids
    constexpr int CPGX = XTile<XT>::kChunks;
    const int nrb = a.I / kGRows;
    const int u = blockIdx.x / nrb, rb = blockIdx.x % nrb;
    // The slot count, the slot's pair count, weight pointers and pair ids (all in the
    // workspace for every slot index of the grid) are read in one round before the exit test.
    const int nu = *a.nu, cnt = a.u_count[u];
    const uint64_t *t = a.u_ptrs + u * 6;
    const uint64_t t0 = t[0], t1 = t[1], t2 = t[2], t3 = t[3];
    const int pid = a.u_pairs[u * a.T + min(static_cast<int>(threadIdx.x), a.T - 1)];
    asm volatile("" ::"s"(nu), "s"(cnt), "s"(t0), "s"(t1), "s"(t2), "s"(t3));
    if (u >= nu) return;  // uniform over the block
    __builtin_amdgcn_sched_barrier(0);  // pid's load ahead of the weight rows: its wait skips them
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int GH = a.Hr >> 5, nch = GH * CPGX;
    const uint32_t rowA = static_cast<uint32_t>(a.Hr >> 1);
    const auto rg = make_rsrc(uniform_ptr(t0), static_cast<uint32_t>(a.I) * rowA);
    const auto rgs = make_rsrc(uniform_ptr(t1), static_cast<uint32_t>(a.I * GH));
    const auto ru = make_rsrc(uniform_ptr(t2), static_cast<uint32_t>(a.I) * rowA);
    const auto rus = make_rsrc(uniform_ptr(t3), static_cast<uint32_t>(a.I * GH));
    // the wave's weight rows, issued before anything is staged
    uint4 wg[kPairsPerWave][GA], wu[kPairsPerWave][GA];
    uint32_t sg[kPairsPerWave][GA], su[kPairsPerWave][GA];
#pragma unroll
    for (int q = 0; q < kPairsPerWave; ++q) {
        const int i = rb * kGRows + wave * kPairsPerWave + q;
#pragma unroll
        for (int v = 0; v < GA; ++v) {
            const int g = v * 64 + lane;
            const bool ok = g < GH;
            const uint32_t off = ok ? static_cast<uint32_t>(i) * rowA + g * 16u : kOobOffset;
            const uint32_t soff = ok ? static_cast<uint32_t>(i * GH + g) : kOobOffset;
            wg[q][v] = buf_load16_nt(rg, off);
            wu[q][v] = buf_load16_nt(ru, off);
            // the scale byte's aligned dword (the byte is picked out where it is used, so no
            // widening of the loaded value is hoisted above the staging)
            sg[q][v] = __builtin_amdgcn_raw_buffer_load_b32(rgs, ok ? soff & ~3u : kOobOffset, 0, 2);
            su[q][v] = __builtin_amdgcn_raw_buffer_load_b32(rus, ok ? soff & ~3u : kOobOffset, 0, 2);
        }
    }
    // the slot's pair ids and the byte offsets of their token rows in x
    if (static_cast<int>(threadIdx.x) < a.T) {
        pair_s[threadIdx.x] = pid;
        tok_s[threadIdx.x] = static_cast<uint32_t>(pid / a.k) * static_cast<uint32_t>(a.Hr * sizeof(XT));
    }
    const auto rx = make_rsrc(a.x, static_cast<uint32_t>(a.T * a.Hr * sizeof(XT)));
    // four staging loads per thread in flight before their stores
    auto stage4 = [&](int c0, int nb, int i0) {
        uint4 v[4];
        int dst[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = i0 + j * 256 + static_cast<int>(threadIdx.x);
            const bool ok = i < nb * nch;
            const int c = ok ? i / nch : 0, cc = ok ? i - c * nch : 0;
            v[j] = buf_load16(rx, ok ? tok_s[c0 + c] + cc * 16u : kOobOffset);
            dst[j] = ok ? c * nch + XTile<XT>::slot(cc / CPGX, cc % CPGX) : -1;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (dst[j] >= 0) smem[dst[j]] = v[j];
    };
    auto compute = [&](int c0, int nb) {
#pragma unroll 1
        for (int c = 0; c < nb; ++c) {
            // the scale bytes are picked out here, not hoisted above the staging (whose
            // stores would then wait for every weight load)
#pragma unroll
            for (int q = 0; q < kPairsPerWave; ++q)
#pragma unroll
                for (int v = 0; v < GA; ++v) asm volatile("" : "+v"(sg[q][v]), "+v"(su[q][v]));
            const uint4 *xs = smem + c * nch;
            float accg[kPairsPerWave], accu[kPairsPerWave];
#pragma unroll
            for (int q = 0; q < kPairsPerWave; ++q) accg[q] = accu[q] = 0.f;
#pragma unroll
            for (int v = 0; v < GA; ++v) {
                const int g = v * 64 + lane;
                if (g < GH) {
                    XChunk<XT> xc[CPGX];
#pragma unroll
                    for (int q = 0; q < CPGX; ++q) xc[q] = reinterpret_cast<const XChunk<XT> *>(xs)[XTile<XT>::slot(g, q)];
#pragma unroll
                    for (int q = 0; q < kPairsPerWave; ++q) {
                        const uint32_t sh =
                            ((static_cast<uint32_t>(rb * kGRows + wave * kPairsPerWave + q) * GH + g) & 3u) * 8u;
                        accg[q] = fmaf(group_dot(wg[q][v], xc), e8m0_to_f32((sg[q][v] >> sh) & 0xffu), accg[q]);
                        accu[q] = fmaf(group_dot(wu[q][v], xc), e8m0_to_f32((su[q][v] >> sh) & 0xffu), accu[q]);
                    }
                }
            }
            const int pair = pair_s[c0 + c];
#pragma unroll
            for (int q = 0; q < kPairsPerWave; ++q) {
                const float gs = wave_sum_to_lane63(accg[q]);
                const float us = wave_sum_to_lane63(accu[q]);
                const int i = rb * kGRows + wave * kPairsPerWave + q;
                if (lane == 63) a.act[static_cast<int64_t>(pair) * a.I + i] = act_fn(gs, us, a.act_kind, a.beta, a.lbeta);
            }
        }
    };
    // The first batch straight-line (a batch of bf16 rows fits in one round of four loads),
    // so the waits before its stores do not cover the weight rows still in flight; further
    // batches (fp32 rows, or more tokens than tb_x) in a loop.
    int nb = min(a.tb_x, cnt);
    __syncthreads();  // pair_s, tok_s
    stage4(0, nb, 0);
#pragma unroll 1
    for (int i0 = 4 * 256; i0 < nb * nch; i0 += 4 * 256) stage4(0, nb, i0);
    __syncthreads();
    compute(0, nb);
#pragma unroll 1
    for (int c0 = a.tb_x; c0 < cnt; c0 += a.tb_x) {
        nb = min(a.tb_x, cnt - c0);
        __syncthreads();  // every wave is done with the previous batch
#pragma unroll 1
        for (int i0 = 0; i0 < nb * nch; i0 += 4 * 256) stage4(c0, nb, i0);
        __syncthreads();
        compute(c0, nb);
    }
}

// ------------------------------------------------------------------ D: down + combine
// A down row is cut into pieces of S elements (S = 32: one group, 16 bytes; S = 16: half a
// group); lane l takes pieces l, l + 64, ... (NP of them) of its wave's RW rows.  A pair's
// act vector is staged chunk-major ([chunk q][piece], plus one zero sink slot), so the lanes
// of a wave read consecutive 16-byte slots.
template <int S, int NP, int RW>
__device__ __forceinline__ void down_body(const MultiArgs &a, int bid) {
    static_assert(S == 16 || S == 32, "a piece is half a group or one group");
    constexpr int ND = S / 8;        // packed dwords per piece
    constexpr int NC = S / 4;        // float4 act chunks per piece
    constexpr int RB = 4 * RW;       // rows per block
    constexpr int NA = S * NP / 16;  // act float4 per thread and pair (I <= S * NP * 64)
    constexpr int AV = NA * 256 + 1; // staged float4 per pair (the last one is the sink)
    extern __shared__ float4 act_s[];  // [tb_act][AV]
    __shared__ int pair_s[kMaxTokens];  // the slot's pair ids
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int nR = (a.Hr + RB - 1) / RB;
    const int u = bid / nR, rr = bid % nR;
    // the slot count, the slot's pair count and down pointers in one round before the exit
    // test (every slot index of the grid has its entries in the workspace)
    const int nu = *a.nu, cnt_u = a.u_count[u];
    const uint64_t t4 = a.u_ptrs[u * 6 + 4], t5 = a.u_ptrs[u * 6 + 5];
    const int pid = a.u_pairs[u * a.T + min(static_cast<int>(threadIdx.x), a.T - 1)];  // the slot's pair ids
    asm volatile("" ::"s"(nu), "s"(cnt_u), "s"(t4), "s"(t5));
    if (u >= nu) return;  // uniform over the block
    __builtin_amdgcn_sched_barrier(0);  // pid's load ahead of the weight rows: its wait skips them
    const int cnt = cnt_u;  // at least one pair in a union slot
    const int GI = a.I >> 5, P = a.I / S;
    const uint32_t rowB = static_cast<uint32_t>(a.I >> 1);
    const int n0 = rr * RB + wave * RW;
    uint32_t wd[RW][NP][ND];
    uint32_t sd[RW][NP];
    {
        const auto rd = make_rsrc(uniform_ptr(t4), static_cast<uint32_t>(a.Hr) * rowB);
        const auto rds = make_rsrc(uniform_ptr(t5), static_cast<uint32_t>(a.Hr * GI));
#pragma unroll
        for (int r = 0; r < RW; ++r)
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const int n = n0 + r, pc = p * 64 + lane;
                const bool ok = n < a.Hr && pc < P;
                const uint32_t off = ok ? static_cast<uint32_t>(n) * rowB + pc * (S / 2u) : kOobOffset;
                if constexpr (S == 32) {
                    const uint4 v = buf_load16_nt(rd, off);
                    wd[r][p][0] = v.x, wd[r][p][1] = v.y, wd[r][p][2] = v.z, wd[r][p][3] = v.w;
                } else {
                    const auto v = __builtin_amdgcn_raw_buffer_load_b64(rd, off, 0, 2);  // nt, as buf_load16_nt
                    wd[r][p][0] = v[0], wd[r][p][1] = v[1];
                }
                // the scale byte's aligned dword (picked out where it is used, so no widening
                // of the loaded value is hoisted above the act staging)
                sd[r][p] = __builtin_amdgcn_raw_buffer_load_b32(
                    rds, ok ? static_cast<uint32_t>(n * GI + pc * S / 32) & ~3u : kOobOffset, 0, 2);
            }
    }
    if (static_cast<int>(threadIdx.x) < a.T) pair_s[threadIdx.x] = pid;
    __syncthreads();
#pragma unroll 1
    for (int c0 = 0; c0 < cnt; c0 += a.tb_act) {
        const int nb = min(a.tb_act, cnt - c0);
        if (c0 > 0) __syncthreads();  // every wave is done with the previous batch
        for (int c = 0; c < nb; ++c) {
            const int pair = pair_s[c0 + c];
            const auto ra = make_rsrc(a.act + static_cast<int64_t>(pair) * a.I, static_cast<uint32_t>(a.I) * 4u);
            float4 *dst = act_s + c * AV;
#pragma unroll
            for (int i = 0; i < NA; ++i) {
                const int ch = i * 256 + static_cast<int>(threadIdx.x);
                const float4 v = __builtin_bit_cast(float4, buf_load16(ra, ch < a.I / 4 ? ch * 16u : kOobOffset));
                dst[ch < a.I / 4 ? (ch % NC) * P + ch / NC : NA * 256] = v;
            }
        }
        __syncthreads();
#pragma unroll 1
        for (int c = 0; c < nb; ++c) {
            const float4 *src = act_s + c * AV;
            float4 av[NP][NC];
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                const int pc = p * 64 + lane;
#pragma unroll
                for (int q = 0; q < NC; ++q) av[p][q] = src[pc < P ? q * P + pc : NA * 256];
            }
            const int pair = pair_s[c0 + c];
            // The packed weights stay packed across the token loop: without this, the
            // compiler hoists their fp4 -> fp32 conversion out of the loop (8 floats per
            // dword) and spills.  An empty asm that claims to modify them keeps it inside.
#pragma unroll
            for (int r = 0; r < RW; ++r)
#pragma unroll
                for (int p = 0; p < NP; ++p) {
#pragma unroll
                    for (int d = 0; d < ND; ++d) asm volatile("" : "+v"(wd[r][p][d]));
                    asm volatile("" : "+v"(sd[r][p]));
                }
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                float acc = 0.f;
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    const uint32_t sh = (static_cast<uint32_t>((n0 + r) * GI + (p * 64 + lane) * S / 32) & 3u) * 8u;
                    acc = fmaf(piece_dot<ND>(wd[r][p], av[p]), e8m0_to_f32((sd[r][p] >> sh) & 0xffu), acc);
                }
                const float tot = wave_sum_to_lane63(acc);
                const int n = n0 + r;
                if (lane == 63 && n < a.Hr) a.yrow[static_cast<int64_t>(pair) * a.Hr + n] = tot;
            }
        }
    }
}

template <int S, int NP, int RW>
__global__ __launch_bounds__(256, 2) void multi_down_kernel(MultiArgs a) {
    down_body<S, NP, RW>(a, static_cast<int>(blockIdx.x));
}

// ------------------------------------------------------------------ C: combine
// One thread per output value (token tk, row n), the token's slots in order.  Every load is
// issued before the sum (slot indices past k are clamped and their terms dropped; a row total
// of a pair that is not live was never written and is selected away, not multiplied by zero).
__global__ __launch_bounds__(256) void multi_combine_kernel(MultiArgs a) {
    const int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (o >= static_cast<int64_t>(a.T) * a.Hr) return;
    const int tk = static_cast<int>(o / a.Hr), n = static_cast<int>(o % a.Hr);
    float v[kMaxTopK], w[kMaxTopK];
    int live[kMaxTopK];
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        const int pair = tk * a.k + min(j, a.k - 1);
        v[j] = a.yrow[static_cast<int64_t>(pair) * a.Hr + n];
        w[j] = a.wts[pair];
        live[j] = a.live[pair];
    }
    float y = a.yadd ? a.yadd[o] : 0.f;
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) y = (j < a.k && live[j]) ? fmaf(w[j], v[j], y) : y;
    if (a.out_bf16)
        static_cast<uint16_t *>(a.out)[o] = f32_to_bf16(y);
    else
        static_cast<float *>(a.out)[o] = y;
}

// ------------------------------------------------------------------ R: dense rows, T tokens
// bf16 row sets [N, K] against T input rows [T, K] (bf16 or fp32) staged in LDS in plain
// 16-byte chunk order, tb tokens at a time (fp32 rows optionally replaced by
// rmsnorm(row) * nw as they are staged); 4 waves per block:
//   plain sets s (blocks in set order): R rows per wave (1 for rows of more than 4096 values,
//       up to 4 for rows of at most 2048), out_s[t * ld_s + n] = W_s[n] . in[t] (+ add_s[...]),
//       fp32 or rounded to bf16
//   the pair set (the last blocks): one (gate, up) row pair per wave,
//       act[t * ld1 + i] = f(G[i] . in[t], U[i] . in[t])
// Products are exact (bf16 x bf16 in v_dot2, bf16 x fp32 as fp32 FMAs), accumulation fp32.
constexpr int kPlainSets = 2;
struct MRowsArgs {
    const void *in;          // [T, K] rows
    int T, K, tb;
    const float *nw;         // not null (fp32 input): stage rmsnorm(row) * nw instead of the row
    float eps;
    const uint16_t *w[kPlainSets];
    int N[kPlainSets], blocks[kPlainSets], ld[kPlainSets], out_bf16[kPlainSets];
    void *out[kPlainSets];
    const float *add[kPlainSets];
    const uint16_t *wg, *wu; // the pair set, rows [N1, K] each
    int N1;
    float *act;
    int ld1;
    int act_kind;
    float beta, lbeta;
    int wv[3];               // persistent form: waves on plain set 0, plain set 1, the pair set
};
constexpr int kRowWaves = 4;
// small enough that LDS allows more blocks per CU than the registers do (three at 133 VGPRs)
constexpr int kLdsBudgetR = 32768;
// 16-byte staging loads per thread and batch for a block of NW waves: kLdsBudgetR for four
// waves, 2 kLdsBudgetR for eight; a batch also always holds one row of 8192 fp32 (32 KB)
constexpr int stage_loads(int NW) { return (NW == kRowWaves ? kLdsBudgetR : 2 * kLdsBudgetR) / (16 * 64 * NW); }
constexpr size_t stage_bytes(int NW) { return static_cast<size_t>(stage_loads(NW)) * 16 * 64 * NW; }

// 8 bf16 weights . 8 bf16 inputs (exact products)
__device__ __forceinline__ float rdot(uint4 w, const uint4 *x, int c, float acc) {
    const uint4 v = x[c];
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.x), __builtin_bit_cast(bf16x2, v.x), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.y), __builtin_bit_cast(bf16x2, v.y), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.z), __builtin_bit_cast(bf16x2, v.z), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.w), __builtin_bit_cast(bf16x2, v.w), acc, false);
    return acc;
}
// 8 bf16 weights . 8 fp32 inputs (the weights widened exactly, fp32 FMAs)
__device__ __forceinline__ float rdot(uint4 w, const float4 *x, int c, float acc) {
    const float4 a = x[2 * c], b = x[2 * c + 1];
    acc = fmaf(__uint_as_float(w.x << 16), a.x, acc);
    acc = fmaf(__uint_as_float(w.x & 0xffff0000u), a.y, acc);
    acc = fmaf(__uint_as_float(w.y << 16), a.z, acc);
    acc = fmaf(__uint_as_float(w.y & 0xffff0000u), a.w, acc);
    acc = fmaf(__uint_as_float(w.z << 16), b.x, acc);
    acc = fmaf(__uint_as_float(w.z & 0xffff0000u), b.y, acc);
    acc = fmaf(__uint_as_float(w.w << 16), b.z, acc);
    acc = fmaf(__uint_as_float(w.w & 0xffff0000u), b.w, acc);
    return acc;
}

// KimiRMSNorm, in place, of nb staged fp32 rows of K values (cpr float4 each):
// row * (1 / sqrt(mean(row^2) + eps)) * nw.  The rows' sums of squares (each thread over its
// chunks in order, then the wave, then the NW waves in order) meet at one barrier, and the
// thread's norm weights load once, all in flight together, for every row.  red: [kMaxTokens][NW].
// CH: the kernel's weight chunks per lane (K <= 512 CH, so a row holds at most 128 CH float4).
template <int NW, int CH>
__device__ __forceinline__ void norm_rows(float4 *x4, int nb, int cpr, int K, const float *nw, float eps,
                                          float (*red)[NW]) {
    constexpr int NT = 64 * NW;
    constexpr int NG = (128 * CH + NT - 1) / NT;  // norm-weight chunks per thread
    const int tid = static_cast<int>(threadIdx.x), lane = tid & 63, wave = tid >> 6;
    const auto rnw = make_rsrc(nw, static_cast<uint32_t>(K) * 4u);
    float4 g[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) g[j] = __builtin_bit_cast(float4, buf_load16(rnw, static_cast<uint32_t>(j * NT + tid) * 16u));
#pragma unroll 1
    for (int c = 0; c < nb; ++c) {
        float ss = 0.f;
        for (int i = tid; i < cpr; i += NT) {
            const float4 v = x4[c * cpr + i];
            ss = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ss))));
        }
        ss = wave_sum_all(ss);
        if (lane == 0) red[c][wave] = ss;
    }
    __syncthreads();
#pragma unroll 1
    for (int c = 0; c < nb; ++c) {
        float tot = red[c][0];
#pragma unroll
        for (int w = 1; w < NW; ++w) tot += red[c][w];
        const float rs = 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            const int i = j * NT + tid;
            if (i < cpr) {
                float4 v = x4[c * cpr + i];
                v.x = v.x * rs * g[j].x, v.y = v.y * rs * g[j].y, v.z = v.z * rs * g[j].z, v.w = v.w * rs * g[j].w;
                x4[c * cpr + i] = v;
            }
        }
    }
    __syncthreads();
}

// IT: input element type (uint16_t = bf16, float); CH: 16-byte weight chunks per lane (K <= 512 CH);
// R: plain rows per wave (narrow rows take several, so one staged batch serves more rows);
// NW: waves per block (4, or 8 to stage inputs of up to twice kLdsBudgetR in one batch).
template <typename IT, int CH, int R, int NW>
__device__ __forceinline__ void rows_body(const MRowsArgs &a, int bid) {
    extern __shared__ uint4 xs[];  // [tb][K * sizeof(IT) / 16]
    __shared__ float red[kMaxTokens][NW];
    using XC = typename std::conditional<std::is_same<IT, float>::value, float4, uint4>::type;
    constexpr int NR = R > 2 ? R : 2;  // weight rows held per wave (a pair needs two)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    int b = bid, s = 0;
    while (s < kPlainSets && b >= a.blocks[s]) b -= a.blocks[s++];
    const bool pair = s == kPlainSets;  // uniform
    const int nrows = pair ? 2 : R;    // rows this wave reduces
    const int n0 = pair ? b * NW + wave : (b * NW + wave) * R;
    const int N = pair ? a.N1 : a.N[s];
    const int nch = a.K >> 3;
    const uint32_t rowb = static_cast<uint32_t>(a.K) * 2u;
    const auto rg = make_rsrc(pair ? a.wg : a.w[s], static_cast<uint32_t>(N) * rowb);
    const auto ru = make_rsrc(a.wu, pair ? static_cast<uint32_t>(N) * rowb : 0u);
    uint4 w[NR][CH];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        // plain: rows n0 + r (r < R); pair: gate row n0 (r = 0) and up row n0 (r = 1)
        const int n = pair ? n0 : n0 + r;
        const bool ok = (pair ? r < 2 : r < R) && n < N;
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int c = u * 64 + lane;
            const uint32_t off = (ok && c < nch) ? static_cast<uint32_t>(n) * rowb + c * 16u : kOobOffset;
            w[r][u] = buf_load16_nt(pair && r == 1 ? ru : rg, off);
        }
    }
    const int cpr = static_cast<int>(a.K * sizeof(IT) / 16);  // 16-byte chunks per input row
    const uint4 *in4 = static_cast<const uint4 *>(a.in);
#pragma unroll 1
    for (int c0 = 0; c0 < a.T; c0 += a.tb) {
        const int nb = min(a.tb, a.T - c0);
        if (c0 > 0) __syncthreads();  // every wave is done with the previous batch
        {
            // every load of the batch issued before the stores (past the end: zeros, no access)
            const auto rin = make_rsrc(in4 + static_cast<int64_t>(c0) * cpr, static_cast<uint32_t>(nb * cpr) * 16u);
            constexpr int kSt = stage_loads(NW);
            uint4 v[kSt];
#pragma unroll
            for (int j = 0; j < kSt; ++j)
                v[j] = buf_load16(rin, static_cast<uint32_t>(j * 64 * NW + static_cast<int>(threadIdx.x)) * 16u);
#pragma unroll
            for (int j = 0; j < kSt; ++j) {
                const int i = j * 64 * NW + static_cast<int>(threadIdx.x);
                if (i < nb * cpr) xs[i] = v[j];
            }
        }
        __syncthreads();
        if constexpr (std::is_same<IT, float>::value) {
            if (a.nw) {
                norm_rows<NW, CH>(reinterpret_cast<float4 *>(xs), nb, cpr, a.K, a.nw, a.eps, red);
            }
        }
#pragma unroll 1
        for (int c = 0; c < nb; ++c) {
            // keep the weights packed inside the token loop (no hoisted widening)
#pragma unroll
            for (int r = 0; r < NR; ++r)
#pragma unroll
                for (int u = 0; u < CH; ++u)
                    asm volatile("" : "+v"(w[r][u].x), "+v"(w[r][u].y), "+v"(w[r][u].z), "+v"(w[r][u].w));
            const XC *xr = reinterpret_cast<const XC *>(xs + c * cpr);
            float acc[NR];
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                float a0 = 0.f, a1 = 0.f;
                if (r < nrows) {
#pragma unroll
                    for (int u = 0; u < CH; ++u) {
                        const int cc = u * 64 + lane;
                        if (cc < nch) {
                            if (u & 1)
                                a1 = rdot(w[r][u], xr, cc, a1);
                            else
                                a0 = rdot(w[r][u], xr, cc, a0);
                        }
                    }
                }
                acc[r] = wave_sum_to_lane63(a0 + a1);
            }
            const int t = c0 + c;
            if (lane == 63) {
                if (pair) {
                    if (n0 < N) a.act[static_cast<int64_t>(t) * a.ld1 + n0] = act_fn(acc[0], acc[1], a.act_kind, a.beta, a.lbeta);
                } else {
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const int n = n0 + r;
                        if (n < N) {
                            const int64_t oi = static_cast<int64_t>(t) * a.ld[s] + n;
                            const float v = a.add[s] ? acc[r] + a.add[s][oi] : acc[r];
                            if (a.out_bf16[s])
                                static_cast<uint16_t *>(a.out[s])[oi] = f32_to_bf16(v);
                            else
                                static_cast<float *>(a.out[s])[oi] = v;
                        }
                    }
                }
            }
        }
    }
}

template <typename IT, int CH, int R, int NW>
__global__ __launch_bounds__(64 * NW) void multi_rows_kernel(MRowsArgs a) {
    rows_body<IT, CH, R, NW>(a, static_cast<int>(blockIdx.x));
}

// D and the 384-expert layer's shared down rows in one launch: blocks [0, nd) run D and the
// rest the four-wave batched form of R over the rows r (fp32 act input), after D's blocks in
// launch order, so they run as D's blocks retire and fill its tail.  As launches of their
// own the shared down rows took 16.8 us for 29 MB (448 blocks, under two per CU) and a
// launch boundary.
template <int S, int NP, int RW, int CH, int R>
__global__ __launch_bounds__(256, 2) void multi_down_rows_kernel(MultiArgs a, MRowsArgs r, int nd) {
    if (static_cast<int>(blockIdx.x) < nd)
        down_body<S, NP, RW>(a, static_cast<int>(blockIdx.x));
    else
        rows_body<float, CH, R, kRowWaves>(r, static_cast<int>(blockIdx.x) - nd);
}

// R in its persistent form, for T input rows that fit in LDS together (up to 128 KB; taken
// for fp32 rows that multi_rows_kernel would stage in three or more batches): a few blocks per CU
// (eight waves each) stage all T rows once (normalised as they are staged when nw is set).
// Every wave of the grid works on one row set for the whole launch -- plain set 0, plain set
// 1 or the pair set, wv[0], wv[1] and wv[2] waves of them, in proportion to the sets' bytes --
// taking the set's rows first, first + stride, ... (stride: the set's wave count), and
// streams them through two register buffers, so one row is in flight while the other is
// reduced against the staged tokens: a plain set's rows alternate between the buffers, a pair
// holds its gate row in one and its up row in the other.  Per row and token the same
// products and the same lane / wave sum order as multi_rows_kernel.
constexpr int kLoopWaves = 8;
constexpr int kStageLoads = 16;                                   // 16-byte loads per thread
constexpr size_t kLoopLdsMax = size_t(kStageLoads) * 16 * 64 * kLoopWaves;  // 128 KB

// res[t] (lane 63) = row . token t for t < T: w one row's 16-byte chunks (chunk c * 64 + lane),
// x the staged tokens (cpr chunks each)
template <typename IT, int CH>
__device__ __forceinline__ void row_dots(uint4 (&w)[CH], const uint4 *x, int cpr, int nch, int lane, int T,
                                         float (&res)[kMaxTokens]) {
    using XC = typename std::conditional<std::is_same<IT, float>::value, float4, uint4>::type;
#pragma unroll
    for (int t = 0; t < kMaxTokens; ++t) {
        if (t >= T) break;
        // keep the weights packed inside the token loop (no hoisted widening)
#pragma unroll
        for (int c = 0; c < CH; ++c) asm volatile("" : "+v"(w[c].x), "+v"(w[c].y), "+v"(w[c].z), "+v"(w[c].w));
        const XC *xr = reinterpret_cast<const XC *>(x + t * cpr);
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int cc = c * 64 + lane;
            if (cc < nch) {
                if (c & 1)
                    a1 = rdot(w[c], xr, cc, a1);
                else
                    a0 = rdot(w[c], xr, cc, a0);
            }
        }
        res[t] = wave_sum_to_lane63(a0 + a1);
    }
}

template <int CH>
__device__ __forceinline__ void load_row(uint4 (&w)[CH], __amdgpu_buffer_rsrc_t rs, int n, int N, uint32_t rowb,
                                         int nch, int lane) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int cc = c * 64 + lane;
        w[c] = buf_load16_nt(rs, (n < N && cc < nch) ? static_cast<uint32_t>(n) * rowb + cc * 16u : kOobOffset);
    }
}

template <typename IT, int CH>
__global__ __launch_bounds__(64 * kLoopWaves) void multi_rows_loop_kernel(MRowsArgs a) {
    extern __shared__ uint4 xs[];  // [T][K * sizeof(IT) / 16]
    __shared__ float red[kMaxTokens][kLoopWaves];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int gw = static_cast<int>(blockIdx.x) * kLoopWaves + wave;
    const int nch = a.K >> 3, T = a.T;
    const uint32_t rowb = static_cast<uint32_t>(a.K) * 2u;
    const int cpr = static_cast<int>(a.K * sizeof(IT) / 16);  // 16-byte chunks per input row

    // this wave's set (wave-uniform) and its rows
    const int v0 = a.wv[0], v1 = a.wv[1], v2 = a.wv[2];
    const bool pair = gw >= v0 + v1;
    const int s = gw < v0 ? 0 : 1;
    const int first = gw < v0 ? gw : (pair ? gw - v0 - v1 : gw - v0);
    const int stride = gw < v0 ? v0 : (pair ? v2 : v1);
    const int N = (gw >= v0 + v1 + v2) ? 0 : (pair ? a.N1 : a.N[s]);  // idle waves: no rows
    const uint32_t bytes = static_cast<uint32_t>(N) * rowb;
    const auto ra = make_rsrc(N ? (pair ? a.wg : a.w[s]) : nullptr, bytes);
    const auto rb = make_rsrc(N ? (pair ? a.wu : a.w[s]) : nullptr, bytes);
    const int step = pair ? stride : 2 * stride;
    int na = first, nb = pair ? first : first + stride;

    uint4 wa[CH], wb[CH];
    load_row<CH>(wa, ra, na, N, rowb, nch, lane);
    load_row<CH>(wb, rb, nb, N, rowb, nch, lane);
    // stage the T input rows: every load issued (past the end: zeros, no access), then the stores
    {
        const int total = T * cpr;
        const auto rin = make_rsrc(a.in, static_cast<uint32_t>(total) * 16u);
        uint4 v[kStageLoads];
#pragma unroll
        for (int j = 0; j < kStageLoads; ++j)
            v[j] = buf_load16(rin, static_cast<uint32_t>(j * 64 * kLoopWaves + static_cast<int>(threadIdx.x)) * 16u);
#pragma unroll
        for (int j = 0; j < kStageLoads; ++j) {
            const int i = j * 64 * kLoopWaves + static_cast<int>(threadIdx.x);
            if (i < total) xs[i] = v[j];
        }
    }
    __syncthreads();
    if constexpr (std::is_same<IT, float>::value) {
        if (a.nw) {
            norm_rows<kLoopWaves, CH>(reinterpret_cast<float4 *>(xs), T, cpr, a.K, a.nw, a.eps, red);
        }
    }

    // plain rows: out[t * ld + n] = dot (+ add), fp32 or bf16
    auto store_plain = [&a, s, lane, T](const float (&res)[kMaxTokens], int n) {
        if (lane != 63) return;
#pragma unroll
        for (int t = 0; t < kMaxTokens; ++t) {
            if (t >= T) break;
            const int64_t oi = static_cast<int64_t>(t) * a.ld[s] + n;
            const float y = a.add[s] ? res[t] + a.add[s][oi] : res[t];
            if (a.out_bf16[s])
                static_cast<uint16_t *>(a.out[s])[oi] = f32_to_bf16(y);
            else
                static_cast<float *>(a.out[s])[oi] = y;
        }
    };
    float ga[kMaxTokens], gb[kMaxTokens];
#pragma unroll 1
    while (na < N) {
        row_dots<IT, CH>(wa, xs, cpr, nch, lane, T, ga);
        if (!pair) store_plain(ga, na);
        load_row<CH>(wa, ra, na + step, N, rowb, nch, lane);
        if (nb >= N) break;
        row_dots<IT, CH>(wb, xs, cpr, nch, lane, T, gb);
        if (pair) {
            if (lane == 63) {
#pragma unroll
                for (int t = 0; t < kMaxTokens; ++t) {
                    if (t >= T) break;
                    a.act[static_cast<int64_t>(t) * a.ld1 + nb] = act_fn(ga[t], gb[t], a.act_kind, a.beta, a.lbeta);
                }
            }
        } else {
            store_plain(gb, nb);
        }
        load_row<CH>(wb, rb, nb + step, N, rowb, nch, lane);
        na += step, nb += step;
    }
}

// Blocks of multi_rows_loop_kernel<IT, CH> resident per CU for lds dynamic bytes (the
// register-bound count, cached per device, capped by the CU's LDS).
template <typename IT, int CH>
int loop_blocks_per_cu(size_t lds, int &cus) {
    constexpr int kDevs = 64;
    static std::atomic<int> cached_occ[kDevs], cached_cus[kDevs], cached_lds[kDevs];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDevs) return 0;
    int occ = cached_occ[dev].load(std::memory_order_relaxed);
    if (!occ) {
        int per_cu = 0, n = 0, l = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, multi_rows_loop_kernel<IT, CH>, 64 * kLoopWaves, 0) !=
                hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipDeviceGetAttribute(&l, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess)
            return 0;
        cached_cus[dev].store(n, std::memory_order_relaxed);
        cached_lds[dev].store(l, std::memory_order_relaxed);
        occ = std::max(1, per_cu);
        cached_occ[dev].store(occ, std::memory_order_relaxed);
    }
    cus = cached_cus[dev].load(std::memory_order_relaxed);
    const size_t l = static_cast<size_t>(cached_lds[dev].load(std::memory_order_relaxed));
    const int by_lds = static_cast<int>(l / (lds + 64 * sizeof(float)));
    return std::max(1, std::min(occ, by_lds));
}

template <typename IT, int CH>
int launch_rows_loop(MRowsArgs &r, size_t lds, hipStream_t st) {
    int cus = 0;
    const int per_cu = loop_blocks_per_cu<IT, CH>(lds, cus);
    if (per_cu <= 0 || cus <= 0) return check_hip(hipErrorInvalidDevice, "moe layer (T tokens): device query");
    // up to 128 KB of dynamic LDS: above the 64 KB default, so opt in once per form
    static const hipError_t lds_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&multi_rows_loop_kernel<IT, CH>),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                                         static_cast<int>(kLoopLdsMax));
    const int rc = check_hip(lds_rc, "moe layer (T tokens): dense rows LDS size");
    if (rc) return rc;
    // the grid's waves split over the sets in proportion to their rows (a pair is two rows),
    // each set at least one wave and at most one wave per unit
    const int64_t units[3] = {r.w[0] ? r.N[0] : 0, r.w[1] ? r.N[1] : 0, r.wg ? r.N1 : 0};
    const int64_t rows = units[0] + units[1] + 2 * units[2];
    const int64_t waves = static_cast<int64_t>(per_cu) * cus * kLoopWaves;
    int total = 0;
    for (int i = 0; i < 3; ++i) {
        const int64_t share = cdiv(waves * units[i] * (i == 2 ? 2 : 1), rows);
        r.wv[i] = units[i] ? static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(share, units[i]))) : 0;
        total += r.wv[i];
    }
    const int blocks = static_cast<int>(cdiv(total, kLoopWaves));
    multi_rows_loop_kernel<IT, CH><<<dim3(static_cast<unsigned>(blocks)), 64 * kLoopWaves, lds, st>>>(r);
    return check_hip(hipGetLastError(), "moe layer (T tokens): dense rows launch");
}

// the eight-wave form of multi_rows_kernel: its static LDS and up to 2 kLdsBudgetR of
// dynamic LDS pass the 64 KB default, so each instance opts in once
template <typename IT, int CH, int R, int NW>
int launch_rows_wide(MRowsArgs &r, dim3 g, size_t lds, hipStream_t st) {
    static const hipError_t lds_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(&multi_rows_kernel<IT, CH, R, NW>),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                                         2 * kLdsBudgetR);
    const int rc = check_hip(lds_rc, "moe layer (T tokens): dense rows LDS size");
    if (rc) return rc;
    multi_rows_kernel<IT, CH, R, NW><<<g, 64 * NW, lds, st>>>(r);
    return check_hip(hipGetLastError(), "moe layer (T tokens): dense rows launch");
}

template <typename IT>
int launch_rows_multi(MRowsArgs &r, hipStream_t st) {
    if (r.nw && !std::is_same<IT, float>::value)
        return set_error(K3_ERR_DTYPE, "moe layer (T tokens): the normalised row input must be fp32");
    if (r.T < 1 || r.T > kMaxTokens) return set_error(K3_ERR_SHAPE, "moe layer (T tokens): %d tokens", r.T);
    const size_t row = static_cast<size_t>(r.K) * sizeof(IT);
    // fp32 rows that the batched kernel would stage in three or more batches (K3's shared
    // down projection at four tokens: 53.7 -> 36.6 us) take the persistent form; elsewhere the
    // batched kernel measured faster (the 384-expert layer's router and shared rows at four
    // tokens: 21.9 against 30 us in the persistent form)
    const size_t in_bytes = static_cast<size_t>(r.T) * row;
    if (std::is_same<IT, float>::value && in_bytes > 2 * static_cast<size_t>(kLdsBudgetR) && in_bytes <= kLoopLdsMax &&
        r.K <= 8192) {
        const int units = (r.w[0] ? r.N[0] : 0) + (r.w[1] ? r.N[1] : 0) + (r.wg ? r.N1 : 0);
        if (units == 0) return K3_OK;
        const size_t lds = static_cast<size_t>(r.T) * row;
        const int ch = static_cast<int>(cdiv(r.K / 8, 64));
        if (ch <= 4) return launch_rows_loop<IT, 4>(r, lds, st);
        if (ch <= 8) return launch_rows_loop<IT, 8>(r, lds, st);
        if (ch <= 14) return launch_rows_loop<IT, 14>(r, lds, st);
        return launch_rows_loop<IT, 16>(r, lds, st);
    }
    const int ch = static_cast<int>(cdiv(r.K / 8, 64));
    if (ch > 16) return set_error(K3_ERR_SHAPE, "moe layer (T tokens): row width %d above 8192", r.K);
    // inputs that need two batches of kLdsBudgetR take one batch in blocks of eight waves where
    // the registers leave room for two such blocks per CU (up to 128 VGPRs: CH <= 8; K3's
    // normalised latent up rows at four tokens: 28 -> 23.6 us).  Wider rows keep four-wave
    // blocks and two batches: one batch in six-wave blocks at three waves per SIMD measured
    // slower (K3's router, latent down and shared gate/up rows at four tokens: 65 -> 90 us).
    const bool wide = ch <= 8 && in_bytes > static_cast<size_t>(kLdsBudgetR) && in_bytes <= stage_bytes(8);
    const int nw = wide ? 8 : kRowWaves;
    r.tb = static_cast<int>(std::max<size_t>(1, std::min<size_t>(r.T, stage_bytes(nw) / row)));
    const int R = ch <= 4 ? 4 : (ch <= 8 ? 2 : 1);
    int blocks = 0;
    for (int s = 0; s < kPlainSets; ++s) {
        r.blocks[s] = r.w[s] ? static_cast<int>(cdiv(r.N[s], nw * R)) : 0;
        blocks += r.blocks[s];
    }
    blocks += r.wg ? static_cast<int>(cdiv(r.N1, nw)) : 0;
    if (blocks == 0) return K3_OK;
    const size_t lds = static_cast<size_t>(r.tb) * row;
    const dim3 g(static_cast<unsigned>(blocks));
    if (wide) {
        if (ch <= 4) return launch_rows_wide<IT, 4, 4, 8>(r, g, lds, st);
        return launch_rows_wide<IT, 8, 2, 8>(r, g, lds, st);
    } else {
        if (ch <= 4)
            multi_rows_kernel<IT, 4, 4, kRowWaves><<<g, 64 * kRowWaves, lds, st>>>(r);
        else if (ch <= 8)
            multi_rows_kernel<IT, 8, 2, kRowWaves><<<g, 64 * kRowWaves, lds, st>>>(r);
        else if (ch <= 14)
            multi_rows_kernel<IT, 14, 1, kRowWaves><<<g, 64 * kRowWaves, lds, st>>>(r);
        else
            multi_rows_kernel<IT, 16, 1, kRowWaves><<<g, 64 * kRowWaves, lds, st>>>(r);
    }
    return check_hip(hipGetLastError(), "moe layer (T tokens): dense rows launch");
}

// ------------------------------------------------------------------ host side
struct MultiWs {
    size_t nu, u_count, u_pairs, live, u_ptrs, act, yrow, total;
};

size_t up256(size_t v) { return (v + 255) & ~size_t(255); }

MultiWs multi_ws_layout(int64_t T, int64_t H, int64_t I, int64_t k) {
    const int64_t P = T * k;
    MultiWs L{};
    size_t o = 0;
    L.nu = o, o += 256;
    L.u_count = o, o += up256(P * 4);
    L.u_pairs = o, o += up256(P * T * 4);
    L.live = o, o += up256(P * 4);
    L.u_ptrs = o, o += up256(P * 6 * 8);
    L.act = o, o += up256(P * I * 4);
    L.yrow = o, o += up256(P * H * 4);
    L.total = o;
    return L;
}

// Rows per D block for the intermediate width's groups GI (as the layer's down launch).
int down_rows(int GI) { return GI <= 64 ? 4 * 14 : (GI <= 96 ? 4 * 7 : 4 * 4); }

int launch_union(MultiArgs &a, hipStream_t st) {
    multi_union_kernel<<<1, 256, 0, st>>>(a);
    return check_hip(hipGetLastError(), "moe routed decode: union launch");
}

template <typename XT>
int launch_gateup(MultiArgs &a, int n_slots, hipStream_t st) {
    const int GH = a.Hr / 32;
    const size_t xrow = static_cast<size_t>(a.Hr) * sizeof(XT);
    a.tb_x = static_cast<int>(std::max<size_t>(1, std::min<size_t>(a.T, kLdsBudgetG / xrow)));
    const int GA = GH <= 64 ? 1 : (GH <= 128 ? 2 : 4);
    const dim3 gg(static_cast<unsigned>(n_slots * (a.I / (4 * g_pairs_per_wave(GA)))));
    const size_t lds_g = static_cast<size_t>(a.tb_x) * xrow;
    if (GH <= 64)
        multi_gateup_kernel<XT, 1><<<gg, 256, lds_g, st>>>(a);
    else if (GH <= 128)
        multi_gateup_kernel<XT, 2><<<gg, 256, lds_g, st>>>(a);
    else
        multi_gateup_kernel<XT, 4><<<gg, 256, lds_g, st>>>(a);
    return check_hip(hipGetLastError(), "moe routed decode: gate/up launch");
}

// D's grid and dynamic LDS for the intermediate width's groups GI (sets a.tb_act)
struct DownShape {
    unsigned blocks;
    size_t lds;
};
DownShape down_shape(MultiArgs &a, int n_slots) {
    const int GI = a.I / 32;
    const int na = GI <= 64 ? 2 : (GI <= 96 ? 3 : 4);  // act float4 per thread and pair
    const size_t per = (static_cast<size_t>(na) * 256 + 1) * 16;
    a.tb_act = static_cast<int>(std::max<size_t>(1, std::min<size_t>(a.T, kLdsBudgetD / per)));
    return {static_cast<unsigned>(n_slots * cdiv(a.Hr, down_rows(GI))), static_cast<size_t>(a.tb_act) * per};
}

int launch_combine(MultiArgs &a, hipStream_t st) {
    const int64_t n_out = static_cast<int64_t>(a.T) * a.Hr;
    multi_combine_kernel<<<dim3(static_cast<unsigned>(cdiv(n_out, 256))), 256, 0, st>>>(a);
    return check_hip(hipGetLastError(), "moe routed decode: combine launch");
}

// D alone
int launch_down_only(MultiArgs &a, int n_slots, hipStream_t st) {
    const DownShape d = down_shape(a, n_slots);
    const int GI = a.I / 32;
    if (GI <= 64)
        multi_down_kernel<32, 1, 14><<<dim3(d.blocks), 256, d.lds, st>>>(a);
    else if (GI <= 96)
        multi_down_kernel<16, 3, 7><<<dim3(d.blocks), 256, d.lds, st>>>(a);
    else
        multi_down_kernel<32, 2, 4><<<dim3(d.blocks), 256, d.lds, st>>>(a);
    return check_hip(hipGetLastError(), "moe routed decode: down launch");
}

// D, then C
int launch_down(MultiArgs &a, int n_slots, hipStream_t st) {
    const int rc = launch_down_only(a, n_slots, st);
    return rc ? rc : launch_combine(a, st);
}

template <int S, int NP, int RW>
void launch_down_rows_ch(MultiArgs &a, MRowsArgs &r, int ch, dim3 g, size_t lds, int nd, hipStream_t st) {
    if (ch <= 4)
        multi_down_rows_kernel<S, NP, RW, 4, 4><<<g, 256, lds, st>>>(a, r, nd);
    else
        multi_down_rows_kernel<S, NP, RW, 8, 2><<<g, 256, lds, st>>>(a, r, nd);
}

// D with the shared down rows r (fp32 act, one plain set) in one launch, then C.  Rows whose
// T inputs do not fit one kLdsBudgetR batch, or wider than 4096 values (whose registers would
// take D to two waves per SIMD), run on their own launch of R first.
int launch_down_rows(MultiArgs &a, int n_slots, MRowsArgs &r, hipStream_t st) {
    const size_t row = static_cast<size_t>(r.K) * sizeof(float);
    const int ch = static_cast<int>(cdiv(r.K / 8, 64));
    if (r.T < 1 || r.T > kMaxTokens || static_cast<size_t>(r.T) * row > static_cast<size_t>(kLdsBudgetR) || ch > 8 ||
        r.w[1] || r.wg || r.nw) {
        const int rc = launch_rows_multi<float>(r, st);
        return rc ? rc : launch_down(a, n_slots, st);
    }
    r.tb = r.T;
    const int R = ch <= 4 ? 4 : 2;
    r.blocks[0] = r.w[0] ? static_cast<int>(cdiv(r.N[0], kRowWaves * R)) : 0;
    r.blocks[1] = 0;
    const DownShape d = down_shape(a, n_slots);
    const dim3 g(d.blocks + static_cast<unsigned>(r.blocks[0]));
    const size_t lds = std::max(d.lds, static_cast<size_t>(r.T) * row);
    const int nd = static_cast<int>(d.blocks), GI = a.I / 32;
    if (GI <= 64)
        launch_down_rows_ch<32, 1, 14>(a, r, ch, g, lds, nd, st);
    else if (GI <= 96)
        launch_down_rows_ch<16, 3, 7>(a, r, ch, g, lds, nd, st);
    else
        launch_down_rows_ch<32, 2, 4>(a, r, ch, g, lds, nd, st);
    const int rc = check_hip(hipGetLastError(), "moe layer (T tokens): down + shared rows launch");
    return rc ? rc : launch_combine(a, st);
}

// The shared expert depends only on x, so the layer entry points run its gate/up and down
// rows on a side stream, beside R, the top-k, U, G and D launches on the caller's stream
// (the few-block top-k and union launches leave most CUs idle).  Two side lanes (a stream and
// a fork / join event pair) per device, created on the device's first such call (default
// priority, non-blocking) and kept until the process ends: one for calls on a stream that is
// not capturing, one for calls under capture.  A stream forked into a capture stays in it
// until that capture ends, so eager calls never use the capture lane; a call under capture
// takes the capture lane when it is idle or already in the same capture, and otherwise (a
// second capture open on the device at once) runs the rows in its own stream.  A call holds
// side_mutex while it enqueues, so calls from several host threads cannot interleave their
// records and waits on the shared events.
struct SideLane {
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex side_mutex;

int new_lane(SideLane &n) {
    int rc = check_hip(hipStreamCreateWithFlags(&n.s, hipStreamNonBlocking), "moe layer (T tokens): side stream");
    if (!rc) rc = check_hip(hipEventCreateWithFlags(&n.fork, hipEventDisableTiming), "moe layer (T tokens): event");
    if (!rc) rc = check_hip(hipEventCreateWithFlags(&n.join, hipEventDisableTiming), "moe layer (T tokens): event");
    return rc;
}

// lane: the side lane for a call on st (hold side_mutex), or null when the lanes do not exist
// yet and st is capturing (creating a stream or an event is not a capturable call), when the
// capture lane belongs to another open capture, or when the environment sets
// K3HIP_SIDE_STREAM=0; the caller then runs the rows in st.
int side_lane(SideLane *&lane, hipStream_t st) {
    constexpr int kDevs = 64;
    static SideLane eager[kDevs], captured[kDevs];
    static const bool enabled = [] {
        const char *e = std::getenv("K3HIP_SIDE_STREAM");
        return !(e && std::strcmp(e, "0") == 0);
    }();
    lane = nullptr;
    if (!enabled) return K3_OK;
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "moe layer (T tokens): device query");
    if (rc) return rc;
    if (dev < 0 || dev >= kDevs) return set_error(K3_ERR_SHAPE, "moe layer (T tokens): device %d", dev);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long id = 0;
    rc = check_hip(hipStreamGetCaptureInfo(st, &cs, &id), "moe layer (T tokens): capture query");
    if (rc) return rc;
    if (cs == hipStreamCaptureStatusNone) {
        if (!eager[dev].s) {
            SideLane e, c;
            rc = new_lane(e);
            if (!rc) rc = new_lane(c);
            if (rc) return rc;
            eager[dev] = e;
            captured[dev] = c;
        }
        lane = &eager[dev];
        return K3_OK;
    }
    if (cs != hipStreamCaptureStatusActive || !captured[dev].s) return K3_OK;
    hipStreamCaptureStatus ls = hipStreamCaptureStatusNone;
    unsigned long long lid = 0;
    rc = check_hip(hipStreamGetCaptureInfo(captured[dev].s, &ls, &lid), "moe layer (T tokens): capture query");
    if (rc) return rc;
    if (ls == hipStreamCaptureStatusNone || (ls == hipStreamCaptureStatusActive && lid == id)) lane = &captured[dev];
    return K3_OK;
}

template <typename XT>
int launch_multi(MultiArgs &a, int n_slots, hipStream_t st) {
    int rc = launch_union(a, st);
    if (!rc) rc = launch_gateup<XT>(a, n_slots, st);
    return rc ? rc : launch_down(a, n_slots, st);
}

// Validation and the MultiArgs of the routed part; the workspace starts at w.
int multi_args(MultiArgs &a, const void *x, int x_dtype, const int32_t *expert_idx, const float *expert_w,
               const void *expert_table, void *out, int out_dtype, int64_t T, int64_t H, int64_t I,
               int64_t n_experts, int64_t top_k, int act_kind, float beta, float linear_beta, char *w,
               const char *what) {
    if (x_dtype != K3_F32 && x_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "%s: x_dtype %d", what, x_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "%s: out_dtype %d", what, out_dtype);
    if (act_kind != K3_ACT_SILU && act_kind != K3_ACT_SITU)
        return set_error(K3_ERR_SHAPE, "%s: act_kind %d", what, act_kind);
    if (T < 1 || T > kMaxTokens)
        return set_error(K3_ERR_SHAPE, "%s: T=%lld must be in 1..%d", what, (long long)T, kMaxTokens);
    if (n_experts <= 0 || n_experts > kMaxExperts || top_k <= 0 || top_k > kMaxTopK || top_k > n_experts)
        return set_error(K3_ERR_SHAPE, "%s: n_experts must be in 1..%d and top_k in 1..min(%d, n_experts)", what,
                         kMaxExperts, kMaxTopK);
    if (H <= 0 || H % 128 || H > 8192 || I <= 0 || I % 128 || I > 4096)
        return set_error(K3_ERR_SHAPE, "%s: H=%lld (multiple of 128, <= 8192) and I=%lld (multiple of 128, <= 4096)",
                         what, (long long)H, (long long)I);
    if (!aligned16(x) || !aligned16(w))
        return set_error(K3_ERR_ALIGN, "%s: x and workspace must be 16-byte aligned", what);
    const MultiWs L = multi_ws_layout(T, H, I, top_k);
    a = MultiArgs{};
    a.x = x;
    a.idx = expert_idx;
    a.wts = expert_w;
    a.table = static_cast<const uint64_t *>(expert_table);
    a.out = out;
    a.T = static_cast<int>(T);
    a.Hr = static_cast<int>(H);
    a.I = static_cast<int>(I);
    a.E = static_cast<int>(n_experts);
    a.k = static_cast<int>(top_k);
    a.P = a.T * a.k;
    a.act_kind = act_kind;
    a.beta = beta;
    a.lbeta = linear_beta;
    a.out_bf16 = out_dtype == K3_BF16;
    a.nu = reinterpret_cast<int32_t *>(w + L.nu);
    a.u_count = reinterpret_cast<int32_t *>(w + L.u_count);
    a.u_pairs = reinterpret_cast<int32_t *>(w + L.u_pairs);
    a.live = reinterpret_cast<int32_t *>(w + L.live);
    a.u_ptrs = reinterpret_cast<uint64_t *>(w + L.u_ptrs);
    a.act = reinterpret_cast<float *>(w + L.act);
    a.yrow = reinterpret_cast<float *>(w + L.yrow);
    return K3_OK;
}

// The whole layer for T tokens: router and shared records after the routed part's (whose
// width is Hr: H, or the latent width of K3's layer, which adds its latent state h and
// routed sum ylat [T, Hr]).
struct LayerMultiWs {
    size_t routed, logits, scores, corrected, idx, w, act_sh, ysh, h, ylat, total;
};

LayerMultiWs layer_multi_layout(int64_t T, int64_t H, int64_t Hr, int64_t I, int64_t Is, int64_t E, int64_t k,
                                bool latent) {
    LayerMultiWs L{};
    size_t o = multi_ws_layout(T, Hr, I, k).total;
    L.routed = 0;
    L.logits = o, o += up256(T * E * 4);
    L.scores = o, o += up256(T * E * 4);
    L.corrected = o, o += up256(T * E * 4);
    L.idx = o, o += up256(T * k * 4);
    L.w = o, o += up256(T * k * 4);
    L.act_sh = o, o += up256(std::max<int64_t>(T * Is, 1) * 4);
    L.ysh = o, o += up256(T * H * 4);
    L.h = o, o += latent ? up256(T * Hr * 4) : 0;
    L.ylat = o, o += latent ? up256(T * Hr * 4) : 0;
    L.total = o;
    return L;
}

}  // namespace
}  // namespace k3

using namespace k3;

extern "C" int64_t k3_moe_routed_workspace_size(int64_t T, int64_t H, int64_t I, int64_t n_experts, int64_t top_k) {
    (void)n_experts;
    if (T <= 0 || H <= 0 || I <= 0 || top_k <= 0) return 0;
    return static_cast<int64_t>(multi_ws_layout(T, H, I, top_k).total);
}

extern "C" int k3_moe_routed_decode(const void *x, int x_dtype, const int32_t *expert_idx, const float *expert_w,
                                    const void *expert_table, void *out, int out_dtype, int64_t T, int64_t H,
                                    int64_t I, int64_t n_experts, int64_t top_k, int act_kind, float beta,
                                    float linear_beta, void *workspace, int64_t workspace_bytes, void *stream) {
    if (!x || !expert_idx || !expert_w || !expert_table || !out || !workspace)
        return set_error(K3_ERR_NULL, "moe routed decode: null pointer");
    MultiArgs a;
    int rc = multi_args(a, x, x_dtype, expert_idx, expert_w, expert_table, out, out_dtype, T, H, I, n_experts, top_k,
                        act_kind, beta, linear_beta, static_cast<char *>(workspace), "moe routed decode");
    if (rc) return rc;
    const MultiWs L = multi_ws_layout(T, H, I, top_k);
    if (workspace_bytes < static_cast<int64_t>(L.total))
        return set_error(K3_ERR_WORKSPACE, "moe routed decode: workspace %lld < %zu bytes",
                         (long long)workspace_bytes, L.total);
    const int n_slots = static_cast<int>(std::min<int64_t>(a.P, n_experts));
    auto st = static_cast<hipStream_t>(stream);
    return x_dtype == K3_BF16 ? launch_multi<uint16_t>(a, n_slots, st) : launch_multi<float>(a, n_slots, st);
}

extern "C" int64_t k3_moe_layer_multi_workspace_size(int64_t T, int64_t H, int64_t I, int64_t shared_I,
                                                     int64_t n_experts, int64_t top_k) {
    if (T <= 0 || H <= 0 || I <= 0 || shared_I < 0 || n_experts <= 0 || top_k <= 0) return 0;
    return static_cast<int64_t>(layer_multi_layout(T, H, H, I, shared_I, n_experts, top_k, false).total);
}

extern "C" int k3_moe_layer_multi_workspace_offsets(int64_t T, int64_t H, int64_t I, int64_t shared_I,
                                                    int64_t n_experts, int64_t top_k, int64_t *offsets) {
    if (!offsets) return set_error(K3_ERR_NULL, "moe layer (T tokens) offsets: null pointer");
    const LayerMultiWs L = layer_multi_layout(T, H, H, I, shared_I, n_experts, top_k, false);
    const size_t v[5] = {L.logits, L.scores, L.corrected, L.idx, L.w};
    for (int i = 0; i < 5; ++i) offsets[i] = static_cast<int64_t>(v[i]);
    return K3_OK;
}

extern "C" int k3_moe_layer_decode_multi(const void *x, int x_dtype, const void *router_w, const void *router_bias,
                                         int route_kind, int renormalize, float scaling, const void *expert_table,
                                         const void *shared_gate, const void *shared_up, const void *shared_down,
                                         void *out, int out_dtype, int64_t T, int64_t H, int64_t I, int64_t shared_I,
                                         int64_t n_experts, int64_t top_k, int act_kind, float beta,
                                         float linear_beta, void *workspace, int64_t workspace_bytes, void *stream) {
    const char *what = "moe layer (T tokens)";
    if (!x || !router_w || !expert_table || !out || !workspace) return set_error(K3_ERR_NULL, "%s: null pointer", what);
    if (route_kind != K3_ROUTE_SOFTMAX && route_kind != K3_ROUTE_SIGMOID_BIAS)
        return set_error(K3_ERR_SHAPE, "%s: route_kind %d", what, route_kind);
    const bool has_shared = shared_gate || shared_up || shared_down;
    if (has_shared && (!shared_gate || !shared_up || !shared_down || shared_I <= 0 || shared_I % 128 ||
                       shared_I > 8192))
        return set_error(K3_ERR_SHAPE, "%s: shared expert needs gate, up and down with shared_I a multiple of 128, "
                         "<= 8192", what);
    if (!aligned16(router_w) || (has_shared && (!aligned16(shared_gate) || !aligned16(shared_up) ||
                                                !aligned16(shared_down))))
        return set_error(K3_ERR_ALIGN, "%s: router and shared weights must be 16-byte aligned", what);
    char *w = static_cast<char *>(workspace);
    const LayerMultiWs L = layer_multi_layout(T, H, H, I, has_shared ? shared_I : 0, n_experts, top_k, false);
    float *logits = reinterpret_cast<float *>(w + L.logits);
    int32_t *idx = reinterpret_cast<int32_t *>(w + L.idx);
    float *wts = reinterpret_cast<float *>(w + L.w);
    MultiArgs a;
    int rc = multi_args(a, x, x_dtype, idx, wts, expert_table, out, out_dtype, T, H, I, n_experts, top_k, act_kind,
                        beta, linear_beta, w, what);
    if (rc) return rc;
    if (workspace_bytes < static_cast<int64_t>(L.total))
        return set_error(K3_ERR_WORKSPACE, "%s: workspace %lld < %zu bytes", what, (long long)workspace_bytes, L.total);
    auto st = static_cast<hipStream_t>(stream);
    const bool bf = x_dtype == K3_BF16;
    // The shared expert (gate/up and down rows, 88 MB at the 384-expert shape) runs on the
    // side stream from the start of the call, beside R (then the router rows alone), the
    // top-k, U and G, and joins before D: four tokens 173.5 -> 171.7 us.  Only its down rows
    // there, forked after R, measured slower (178.4 -> 180.3 us); without a side lane (see
    // side_lane) they run as extra blocks of D's launch.
    std::unique_lock<std::mutex> lock(side_mutex, std::defer_lock);
    SideLane *side = nullptr;
    if (has_shared) {
        lock.lock();
        rc = side_lane(side, st);
        if (rc) return rc;
    }
    // R: router logits [T, E] (and the shared gate/up act [T, shared_I] without a side stream)
    MRowsArgs r{};
    r.in = x;
    r.T = a.T;
    r.K = a.Hr;
    r.w[0] = static_cast<const uint16_t *>(router_w);
    r.N[0] = a.E;
    r.out[0] = logits;
    r.ld[0] = a.E;
    float *act_sh = reinterpret_cast<float *>(w + L.act_sh);
    MRowsArgs g{};  // the shared gate/up pairs on x
    g.in = x;
    g.T = a.T;
    g.K = a.Hr;
    g.wg = static_cast<const uint16_t *>(shared_gate);
    g.wu = static_cast<const uint16_t *>(shared_up);
    g.N1 = static_cast<int>(shared_I);
    g.act = act_sh;
    g.ld1 = static_cast<int>(shared_I);
    g.act_kind = act_kind;
    g.beta = beta;
    g.lbeta = linear_beta;
    MRowsArgs d{};  // the shared down rows [H, shared_I] against the fp32 act -> [T, H], added in C
    d.in = act_sh;
    d.T = a.T;
    d.K = static_cast<int>(shared_I);
    d.w[0] = static_cast<const uint16_t *>(shared_down);
    d.N[0] = a.Hr;
    d.out[0] = w + L.ysh;
    d.ld[0] = a.Hr;
    if (has_shared) a.yadd = reinterpret_cast<const float *>(w + L.ysh);
    if (side) {
        // R is enqueued before the side stream's launches (same dependencies): a graph
        // replay then dispatches R first (see the latent entry point)
        rc = check_hip(hipEventRecord(side->fork, st), "moe layer (T tokens): fork");
        if (!rc) rc = bf ? launch_rows_multi<uint16_t>(r, st) : launch_rows_multi<float>(r, st);
        if (!rc) rc = check_hip(hipStreamWaitEvent(side->s, side->fork, 0), "moe layer (T tokens): fork");
        if (!rc) rc = bf ? launch_rows_multi<uint16_t>(g, side->s) : launch_rows_multi<float>(g, side->s);
        if (!rc) rc = launch_rows_multi<float>(d, side->s);
        const int jr = check_hip(hipEventRecord(side->join, side->s), "moe layer (T tokens): join");
        if (!rc) rc = jr;
    } else {
        if (has_shared) {
            r.wg = g.wg, r.wu = g.wu, r.N1 = g.N1, r.act = g.act, r.ld1 = g.ld1;
            r.act_kind = act_kind, r.beta = beta, r.lbeta = linear_beta;
        }
        rc = bf ? launch_rows_multi<uint16_t>(r, st) : launch_rows_multi<float>(r, st);
    }
    // the batched top-k on those logits (softmax / sigmoid + bias, renormalised, scaled)
    if (!rc)
        rc = k3_moe_topk(logits, a.E, a.T, a.E, static_cast<const float *>(router_bias), route_kind, renormalize,
                         scaling, a.k, idx, wts, reinterpret_cast<float *>(w + L.scores),
                         reinterpret_cast<float *>(w + L.corrected), stream);
    const int n_slots = static_cast<int>(std::min<int64_t>(a.P, n_experts));
    if (!rc) rc = launch_union(a, st);
    if (!rc) rc = bf ? launch_gateup<uint16_t>(a, n_slots, st) : launch_gateup<float>(a, n_slots, st);
    if (side) {
        // joined before D rather than before C (the side stream's work ended long before G
        // does): 170.5 -> 170.0 us
        const int jr = check_hip(hipStreamWaitEvent(st, side->join, 0), "moe layer (T tokens): join");
        if (!rc) rc = jr;  // an error after the fork still joins
        if (!rc) rc = launch_down_only(a, n_slots, st);
        return rc ? rc : launch_combine(a, st);
    }
    if (rc) return rc;
    if (has_shared) return launch_down_rows(a, n_slots, d, st);
    return launch_down(a, n_slots, st);
}

extern "C" int64_t k3_moe_latent_layer_multi_workspace_size(int64_t T, int64_t H, int64_t latent, int64_t I,
                                                            int64_t shared_I, int64_t n_experts, int64_t top_k) {
    if (T <= 0 || H <= 0 || latent <= 0 || I <= 0 || shared_I < 0 || n_experts <= 0 || top_k <= 0) return 0;
    return static_cast<int64_t>(layer_multi_layout(T, H, latent, I, shared_I, n_experts, top_k, true).total);
}

extern "C" int k3_moe_latent_layer_multi_workspace_offsets(int64_t T, int64_t H, int64_t latent, int64_t I,
                                                           int64_t shared_I, int64_t n_experts, int64_t top_k,
                                                           int64_t *offsets) {
    if (!offsets) return set_error(K3_ERR_NULL, "moe latent layer (T tokens) offsets: null pointer");
    const LayerMultiWs L = layer_multi_layout(T, H, latent, I, shared_I, n_experts, top_k, true);
    const size_t v[5] = {L.logits, L.scores, L.corrected, L.idx, L.w};
    for (int i = 0; i < 5; ++i) offsets[i] = static_cast<int64_t>(v[i]);
    return K3_OK;
}

extern "C" int k3_moe_latent_layer_decode_multi(const void *x, int x_dtype, const void *router_w,
                                                const void *router_bias, int renormalize, float scaling,
                                                const void *expert_table, const void *latent_down,
                                                const void *latent_up, const void *latent_norm, float eps,
                                                const void *shared_gate, const void *shared_up,
                                                const void *shared_down, void *out, int out_dtype, int64_t T,
                                                int64_t H, int64_t latent, int64_t I, int64_t shared_I,
                                                int64_t n_experts, int64_t top_k, int act_kind, float beta,
                                                float linear_beta, void *workspace, int64_t workspace_bytes,
                                                void *stream) {
    const char *what = "moe latent layer (T tokens)";
    if (!x || !router_w || !expert_table || !latent_down || !latent_up || !latent_norm || !out || !workspace)
        return set_error(K3_ERR_NULL, "%s: null pointer", what);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "%s: out_dtype %d", what, out_dtype);
    if (H <= 0 || H % 128 || H > 8192)
        return set_error(K3_ERR_SHAPE, "%s: H=%lld must be a multiple of 128, <= 8192", what, (long long)H);
    const bool has_shared = shared_gate || shared_up || shared_down;
    if (has_shared && (!shared_gate || !shared_up || !shared_down || shared_I <= 0 || shared_I % 128 ||
                       shared_I > 8192))
        return set_error(K3_ERR_SHAPE, "%s: shared expert needs gate, up and down with shared_I a multiple of 128, "
                         "<= 8192", what);
    if (!aligned16(router_w) || !aligned16(latent_down) || !aligned16(latent_up) || !aligned16(latent_norm) ||
        (has_shared && (!aligned16(shared_gate) || !aligned16(shared_up) || !aligned16(shared_down))))
        return set_error(K3_ERR_ALIGN, "%s: dense weights must be 16-byte aligned", what);
    char *w = static_cast<char *>(workspace);
    const LayerMultiWs L = layer_multi_layout(T, H, latent, I, has_shared ? shared_I : 0, n_experts, top_k, true);
    int32_t *idx = reinterpret_cast<int32_t *>(w + L.idx);
    float *wts = reinterpret_cast<float *>(w + L.w);
    void *h = w + L.h;
    float *ylat = reinterpret_cast<float *>(w + L.ylat);
    MultiArgs a;
    // the routed part reads h (x's dtype) and writes the fp32 routed sum ylat
    int rc = multi_args(a, h, x_dtype, idx, wts, expert_table, ylat, K3_F32, T, latent, I, n_experts, top_k, act_kind,
                        beta, linear_beta, w, what);
    if (rc) return rc;
    if (workspace_bytes < static_cast<int64_t>(L.total))
        return set_error(K3_ERR_WORKSPACE, "%s: workspace %lld < %zu bytes", what, (long long)workspace_bytes, L.total);
    auto st = static_cast<hipStream_t>(stream);
    const bool bf = x_dtype == K3_BF16;
    float *logits = reinterpret_cast<float *>(w + L.logits);
    float *act_sh = reinterpret_cast<float *>(w + L.act_sh);
    float *ysh = reinterpret_cast<float *>(w + L.ysh);
    std::unique_lock<std::mutex> lock(side_mutex, std::defer_lock);
    SideLane *side = nullptr;
    if (has_shared) {
        lock.lock();
        rc = side_lane(side, st);
        if (rc) return rc;
    }
    // R1 on x: router logits, h = W_down x (bf16 for a bf16 x, as the reference's bf16
    // matmul; fp32 for an fp32 x), and the shared gate/up act unless the side stream takes it
    MRowsArgs r{};
    r.in = x;
    r.T = a.T;
    r.K = static_cast<int>(H);
    r.w[0] = static_cast<const uint16_t *>(router_w);
    r.N[0] = a.E;
    r.out[0] = logits;
    r.ld[0] = a.E;
    r.w[1] = static_cast<const uint16_t *>(latent_down);
    r.N[1] = a.Hr;
    r.out[1] = h;
    r.ld[1] = a.Hr;
    r.out_bf16[1] = bf;
    MRowsArgs g{};  // the shared gate/up pairs on x
    g.in = x;
    g.T = a.T;
    g.K = static_cast<int>(H);
    g.wg = static_cast<const uint16_t *>(shared_gate);
    g.wu = static_cast<const uint16_t *>(shared_up);
    g.N1 = static_cast<int>(shared_I);
    g.act = act_sh;
    g.ld1 = static_cast<int>(shared_I);
    g.act_kind = act_kind;
    g.beta = beta;
    g.lbeta = linear_beta;
    MRowsArgs d{};  // the shared down rows on the shared act
    d.in = act_sh;
    d.T = a.T;
    d.K = static_cast<int>(shared_I);
    d.w[0] = static_cast<const uint16_t *>(shared_down);
    d.N[0] = static_cast<int>(H);
    d.out[0] = ysh;
    d.ld[0] = static_cast<int>(H);
    if (side) {
        // the whole shared expert (264 MB at K3's shapes) on the side stream from the start of
        // the call, beside R1, the top-k, U, G and D; R3 adds its output.  K3's four-token step
        // 338 -> 325 us with the shared down rows alone there (forked after R1), 322 -> 318 us
        // with the gate/up rows too; forked after U (beside G and D only): 337 us.  R1 is
        // enqueued after the fork record and before the side stream's wait and launches (the
        // same dependencies): a graph replay dispatches nodes in the order they were
        // captured, and with the side stream's launches captured first R1 started about 6 us
        // after them (319 -> 304.5 us)
        rc = check_hip(hipEventRecord(side->fork, st), "moe layer (T tokens): fork");
        if (!rc) rc = bf ? launch_rows_multi<uint16_t>(r, st) : launch_rows_multi<float>(r, st);
        if (!rc) rc = check_hip(hipStreamWaitEvent(side->s, side->fork, 0), "moe layer (T tokens): fork");
        if (!rc) rc = bf ? launch_rows_multi<uint16_t>(g, side->s) : launch_rows_multi<float>(g, side->s);
        if (!rc) rc = launch_rows_multi<float>(d, side->s);
        const int jr = check_hip(hipEventRecord(side->join, side->s), "moe layer (T tokens): join");
        if (!rc) rc = jr;
    } else {
        if (has_shared) {
            r.wg = g.wg, r.wu = g.wu, r.N1 = g.N1, r.act = g.act, r.ld1 = g.ld1;
            r.act_kind = act_kind, r.beta = beta, r.lbeta = linear_beta;
        }
        rc = bf ? launch_rows_multi<uint16_t>(r, st) : launch_rows_multi<float>(r, st);
        if (!rc && has_shared) rc = launch_rows_multi<float>(d, st);
    }
    // sigmoid + bias routing (moe.py:65-76) on the logits
    if (!rc)
        rc = k3_moe_topk(logits, a.E, a.T, a.E, static_cast<const float *>(router_bias), K3_ROUTE_SIGMOID_BIAS,
                         renormalize, scaling, a.k, idx, wts, reinterpret_cast<float *>(w + L.scores),
                         reinterpret_cast<float *>(w + L.corrected), stream);
    const int n_slots = static_cast<int>(std::min<int64_t>(a.P, n_experts));
    if (!rc) rc = launch_union(a, st);
    if (!rc) rc = bf ? launch_gateup<uint16_t>(a, n_slots, st) : launch_gateup<float>(a, n_slots, st);
    if (!rc) rc = launch_down(a, n_slots, st);
    if (side) {
        const int jr = check_hip(hipStreamWaitEvent(st, side->join, 0), "moe latent layer (T tokens): join");
        if (!rc) rc = jr;  // an error after the fork still joins
    }
    if (rc) return rc;
    // R3: out = W_up rmsnorm(ylat) * norm (+ the shared output), in out_dtype
    MRowsArgs u{};
    u.in = ylat;
    u.T = a.T;
    u.K = a.Hr;
    u.nw = static_cast<const float *>(latent_norm);
    u.eps = eps;
    u.w[0] = static_cast<const uint16_t *>(latent_up);
    u.N[0] = static_cast<int>(H);
    u.out[0] = out;
    u.ld[0] = static_cast<int>(H);
    u.out_bf16[0] = out_dtype == K3_BF16;
    u.add[0] = has_shared ? ysh : nullptr;
    return launch_rows_multi<float>(u, st);
}
