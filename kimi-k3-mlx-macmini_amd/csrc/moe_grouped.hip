// Grouped routed-expert FFN for many tokens (prefill) on native MXFP4 MFMA: every routed
// (token, slot) pair is grouped by expert and each expert runs as a GEMM with M = its token
// count, so each expert's MXFP4 weights stream from HBM once per 64-row tile instead of
// once per token.
//
// Reference: LatentMoE.__call__ (air_llm/models/kimi_k3/moe.py:110-132; k3ref
// k3ref/layers.py:241-261): for each distinct routed expert, gather its tokens, run
// expert_forward, scale by the gate weight and add into y.  The reference loops over
// experts on the host; here:
//
//   count    block e counts the pairs routed to expert e                      -> counts[E]
//   plan     one block: exclusive scan of the counts (segment bases) and the list of
//            64-row tiles (expert, first row) of every non-empty expert
//   place    block e writes its pairs, in (token, slot) order, into perm[base_e ...]
//   quant_x  x -> E4M3 terms, one E8M0 scale per 32 elements per term: bf16 x as two,
//            x = 2^e1 t1 + 2^e2 t2, exact for every element within 2^13 of its block's max;
//            fp32 x as three (about 12 bits, as act)
//   gateup   block (tile, 128 intermediate indices): v_mfma_scale_f32_16x16x128_f8f6f4 with
//            the expert's MXFP4 rows as the FP4 A operand and their E8M0 bytes as the A
//            scales (no decode), the x terms as the FP8 B operand; act = f(gate, up) in
//            fp32, split in registers into three E4M3 terms per 32 (about 12 bits)
//   down     block (tile, 256 output rows): the same MFMA over the three act terms
//            -> fp32 rows per (token, slot) pair
//   combine  y[t] = sum_slot w[t, slot] * y_pair[t, slot], slots in order
//
// Deterministic: no atomics, fixed summation orders everywhere.
//
// Operand layout of v_mfma_scale_f32_16x16x128_f8f6f4 with FP4 A (cbsz 4) and FP8 E4M3 B
// (blgp 0), as measured on gfx950:
//   A   lane l: weight row l%16, the 32 elements of K block l/16 (of the instruction's 128),
//       element j in nibble j, low nibble first -- the MXFP4 byte order, loaded verbatim
//   B   lane l: column l%16; with g = l/16, bytes 0-15 hold elements 16(g%2)..16(g%2)+15 of
//       K block g/2 and bytes 16-31 the same elements of K block 2+g/2
//   scale_a / scale_b of lane l: row / column l%16, K block l/16; op_sel picks the byte
//   C   lane l, register v: row 4(l/16)+v, column l%16
// The 128-element dot is accumulated about 12 bits below its largest product (unbiased
// rounding, measured), then added into the fp32 C.
//
// K runs in super-steps of 256: a lane's 32-byte A load covers blocks 2q, 2q+1 (q = l/16)
// and MFMA m in {0, 1} uses block 2q+m, so MFMA m's K block q' is super-step block 2q'+m.
// B rows are therefore stored in "MX-B" order: per super-step, sixteen 16-byte pieces
// p = (m*2 + h)*4 + g, piece p holding elements 16(g%2)..+15 of block 4h + 2(g/2) + m.  The
// B operand of (m, lane) is then pieces (m, h=0, g) and (m, h=1, g) of its row, and its
// scale is byte 2g+m of the row's eight block scales (natural order).
#include <algorithm>

#include "k3_common.h"
#include "moe_common.h"

namespace k3 {
namespace {

constexpr int kTM = 64;        // grouped rows (tokens) per tile: four 16-column B tiles
constexpr int kSS = 256;       // K elements per super-step
constexpr int kThreads = 256;  // 4 waves

typedef int i32x8 __attribute__((ext_vector_type(8)));

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

// Stable compaction of the pairs equal to `e`, by one 1024-thread block: wave w scans the
// contiguous range [w * span, (w + 1) * span) of the pairs with ballots, kScanLoads ids per
// lane in flight at once and no barrier inside the scan; the waves' hit counts meet in LDS
// once, and the writing pass places wave w's hits after those of waves 0 .. w - 1, so the
// pairs keep their ascending order.  (One barrier per 256 pairs, one id load per lane at a
// time, ran 28-34 us at 16,384 pairs.)  Returns the block's total.
constexpr int kScanThreads = 1024;
constexpr int kScanWaves = kScanThreads / 64;
constexpr int kScanLoads = 16;  // ids per lane in flight
template <bool WRITE>
__device__ int scan_expert(const GroupArgs &g, int e, int32_t *out) {
    __shared__ int wcnt[kScanWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int span = (g.P + kScanWaves * 64 - 1) / (kScanWaves * 64) * 64;  // a multiple of 64
    const int lo = wave * span, hi = min(g.P, lo + span);
    // one pass over the wave's range; hits(u, mask) for each group of 64 pairs in order
    auto pass = [&](auto &&hits) {
        for (int p0 = lo; p0 < hi; p0 += 64 * kScanLoads) {
            int v[kScanLoads];
#pragma unroll
            for (int u = 0; u < kScanLoads; ++u) {
                const int p = p0 + 64 * u + lane;
                v[u] = p < hi ? g.idx[p] : -1;
            }
#pragma unroll
            for (int u = 0; u < kScanLoads; ++u) hits(p0 + 64 * u + lane, v[u] == e, __ballot(v[u] == e));
        }
    };
    int cnt = 0;
    pass([&](int, bool, uint64_t m) { cnt += __popcll(m); });
    if (lane == 0) wcnt[wave] = cnt;
    __syncthreads();
    int before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kScanWaves; ++w) {
        before += w < wave ? wcnt[w] : 0;
        total += wcnt[w];
    }
    if (WRITE) {
        pass([&](int p, bool hit, uint64_t m) {
            if (hit) out[before + __popcll(m & ((1ull << lane) - 1ull))] = p;
            before += __popcll(m);
        });
    }
    return total;
}

__global__ __launch_bounds__(kScanThreads) void group_count_kernel(GroupArgs g) {
    const int n = scan_expert<false>(g, blockIdx.x, nullptr);
    if (threadIdx.x == 0) g.counts[blockIdx.x] = n;
}

__global__ __launch_bounds__(kScanThreads) void group_place_kernel(GroupArgs g) {
    scan_expert<true>(g, blockIdx.x, g.perm + g.base[blockIdx.x]);
}

// One block of 1024 threads: segment bases and the tile list (E <= 1024).
__global__ __launch_bounds__(1024) void group_plan_kernel(GroupArgs g) {
    __shared__ int sc[1024], st[1024];
    const int e = threadIdx.x;
    const int c = e < g.E ? g.counts[e] : 0;
    sc[e] = c;
    st[e] = (c + kTM - 1) / kTM;
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
        const int t0 = st[e] - (c + kTM - 1) / kTM;
        for (int j = 0; j * kTM < c; ++j) {
            if (t0 + j < g.max_tiles) {
                g.tile_e[t0 + j] = e;
                g.tile_m0[t0 + j] = j * kTM;
            }
        }
    }
    if (e == 1023) *g.n_tiles = min(st[1023], g.max_tiles);
}

// ------------------------------------------------------------------ E4M3 / E8M0 terms
// Exponent e of the block scale 2^e for a block whose largest magnitude is amax, chosen so
// amax / 2^e lies in [128, 256) (below E4M3's 448); clamped to the E8M0 range.
__device__ __forceinline__ int block_exp(float amax) {
    const int ea = static_cast<int>((__float_as_uint(amax) >> 23) & 0xffu) - 127;
    return max(ea - 7, -127);
}

// E4M3 (OCP, bias 7) code of x, |x| < 256, rounded to nearest even; q receives its value.
__device__ __forceinline__ uint32_t e4m3_rne(float x, float &q) {
    const float a = fabsf(x);
    uint32_t code;
    float v;
    if (a < 0.015625f) {  // subnormals: multiples of 2^-9 (rounding up to 8 gives 2^-6, code 8)
        const float m = rintf(a * 512.f);
        code = static_cast<uint32_t>(m);
        v = m * 0.001953125f;
    } else {              // normals: keep 3 mantissa bits, the carry runs into the exponent
        uint32_t b = __float_as_uint(a);
        b += 0x7ffffu + ((b >> 20) & 1u);
        b &= 0xfff00000u;
        v = __uint_as_float(b);
        code = (b >> 20) - 960u;  // ((exp - 127 + 7) << 3) | mantissa
    }
    const uint32_t s = __float_as_uint(x) >> 31;
    q = s ? -v : v;
    return code | (s << 7);
}

// Byte offset, inside one row in MX-B order, of the 16-element half `half` of K block b.
__device__ __forceinline__ uint32_t mxb_offset(uint32_t b, uint32_t half) {
    const uint32_t bb = b & 7u, m = bb & 1u, h = bb >> 2, g = ((bb >> 1) & 1u) * 2u + half;
    return (b >> 3) * kSS + ((m * 2u + h) * 4u + g) * 16u;
}

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

// ------------------------------------------------------------------ quant_x
struct QxArgs {
    const void *x;        // [T, H] bf16 (two terms) or fp32 (three terms)
    uint8_t *x8;          // [TERMS][T][Hpad] E4M3 codes, MX-B order
    uint8_t *xs;          // [TERMS][T][Hpad / 32] E8M0
    int T, H, Hpad;
    uint32_t term, sterm; // bytes per term of x8 / xs
};

// One thread per 16-element half block; the two halves of a block are adjacent lanes.
// bf16 x is the exact sum of its two terms; fp32 x keeps about 12 bits in three (as act).
template <bool F32>
__global__ __launch_bounds__(256) void quant_x_kernel(QxArgs a) {
    constexpr int TERMS = F32 ? 3 : 2;
    const int halves = a.H >> 4;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    const bool ok = idx < a.T * halves;
    const int t = ok ? idx / halves : 0, hh = ok ? idx % halves : 0;
    float v[16];
    if (ok && F32) {
        const float4 *src = reinterpret_cast<const float4 *>(static_cast<const float *>(a.x) +
                                                             static_cast<int64_t>(t) * a.H + hh * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 f = src[i];
            v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
        }
    } else if (ok) {
        const uint4 *src = reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(a.x) +
                                                           static_cast<int64_t>(t) * a.H + hh * 16);
        const uint4 u0 = src[0], u1 = src[1];
        const uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = 0.f;
    }
    const uint32_t row8 = static_cast<uint32_t>(t) * a.Hpad + mxb_offset(hh >> 1, hh & 1);
    const uint32_t rows = static_cast<uint32_t>(t) * (a.Hpad >> 5) + (hh >> 1);
#pragma unroll
    for (int term = 0; term < TERMS; ++term) {
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
        amax = fmaxf(amax, shfl_xor_f(amax, 1));
        const int e = block_exp(amax);
        uint32_t c[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            float q;
            c[i >> 2] |= e4m3_rne(ldexpf(v[i], -e), q) << (8 * (i & 3));
            v[i] -= ldexpf(q, e);
        }
        if (ok) {
            *reinterpret_cast<uint4 *>(a.x8 + term * a.term + row8) = make_uint4(c[0], c[1], c[2], c[3]);
            if ((hh & 1) == 0) a.xs[term * a.sterm + rows] = static_cast<uint8_t>(e + 127);
        }
    }
}

// ------------------------------------------------------------------ grouped MFMA GEMMs
struct MxArgs {
    const uint8_t *b8;       // B terms [TERMS][rows][Kpad], MX-B order
    const uint8_t *bs;       // B scales [TERMS][rows][Kpad / 32]
    uint32_t b_term, bs_term;
    const uint64_t *table;   // [E][6] expert pointers
    const int32_t *counts, *base, *perm, *tile_e, *tile_m0, *n_tiles;
    uint8_t *a8, *as;        // gate/up output: act terms [3][P][Ipad], scales [3][P][Ipad / 32]
    uint32_t a_term, as_term;
    int Ipad;
    float *ypair;            // down output [P, H]: row = pair id
    int K, Kpad, N;          // reduction length, its padded row length, weight rows of one projection
    int NT, tile_major;      // weight-row blocks; block order (see mx_gemm_kernel)
    int top_k, max_tiles, act_kind;
    float beta, lbeta;
};

template <int M>
__device__ __forceinline__ f32x4 mfma_fp4_fp8(const uint4 &a, const uint4 &b0, const uint4 &b1, f32x4 c,
                                              uint32_t sa, uint32_t sb) {
    const i32x8 av = {static_cast<int>(a.x), static_cast<int>(a.y), static_cast<int>(a.z), static_cast<int>(a.w),
                      0, 0, 0, 0};
    const i32x8 bv = {static_cast<int>(b0.x), static_cast<int>(b0.y), static_cast<int>(b0.z), static_cast<int>(b0.w),
                      static_cast<int>(b1.x), static_cast<int>(b1.y), static_cast<int>(b1.z), static_cast<int>(b1.w)};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, c, 4, 0, M, static_cast<int>(sa), M,
                                                            static_cast<int>(sb));
}

// DOWN == false: gate/up + activation.  Wave w owns the 32 intermediate indices
// [i0 + 32 w, +32): A tiles j = 0, 1 are their gate rows and j = 2, 3 their up rows, so the
// activation of a (token, index) pair meets both products in one lane.
// DOWN == true: wave w owns 64 output rows [n0 + 64 w, +64) of W_down, B = the act terms.
// TERMS: E4M3 terms of B (x: 2 for bf16, 3 for fp32; act: 3).
template <bool DOWN, int TERMS>
__global__ __launch_bounds__(kThreads, 1) void mx_gemm_kernel(MxArgs a) {
    // two LDS tiles of B: [buffer][ct][term][piece][column] 16-byte pieces, then
    // [buffer][ct][term][column][block pair] scale pairs
    extern __shared__ uint4 smem[];
    constexpr int kXT = 4 * TERMS * 16 * 16;  // uint4 per tile
    constexpr int kST = 4 * TERMS * 16 * 4;   // uint16 per scale tile
    uint16_t *const ssm = reinterpret_cast<uint16_t *>(smem + 2 * kXT);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Block order (block b runs on XCD b % 8).  Row-block major (gate/up): consecutive blocks
    // on one XCD take consecutive tiles of one weight-row block, so the tiles of a hot expert
    // stream the same weight rows together and share them in L2.  Tile major (down): XCD x
    // owns tiles x, x + 8, ... and runs all row blocks of one tile together, so they share
    // that tile's B rows (its act terms) in L2.  Measured on the 2048-token Zipf prefill:
    // tile major is 8% faster for down and 5-12% slower for gate/up, where a hot expert's
    // weight rows then stream once per XCD; groups of several tiles x row blocks per XCD were
    // slower for both.
    int tile, nt;
    if (a.tile_major) {
        const int li = blockIdx.x >> 3;
        tile = (blockIdx.x & 7) + 8 * (li / a.NT), nt = li % a.NT;
    } else {
        const int nb = static_cast<int>(gridDim.x);
        const int w = (nb & 7) == 0 ? (blockIdx.x & 7) * (nb >> 3) + (blockIdx.x >> 3) : blockIdx.x;
        tile = w % a.max_tiles, nt = w / a.max_tiles;
    }
    if (tile >= *a.n_tiles || nt >= a.NT) return;
    const int e = a.tile_e[tile], m0 = a.tile_m0[tile];
    const int rows = min(kTM, a.counts[e] - m0);
    const int pos0 = a.base[e] + m0;  // grouped row of the tile's first token
    const int nct = (rows + 15) >> 4;
    const uint64_t *ptr = a.table + static_cast<int64_t>(e) * 6;
    const int KB = a.K >> 5;
    const int NS = a.Kpad / kSS;
    const int r16 = lane & 15, q = lane >> 4;

    // ---- A: four 16-row tiles per wave, 32 bytes + 2 scale bytes per lane per super-step,
    // in a ring of four super-steps (loads run three super-steps ahead of their MFMAs)
    const uint32_t rowA = static_cast<uint32_t>(a.K >> 1);
    __amdgpu_buffer_rsrc_t ra[2], rsa[2];
    {
        const int p0 = DOWN ? 4 : 0;
        ra[0] = make_rsrc(reinterpret_cast<const void *>(ptr[p0]), static_cast<uint32_t>(a.N) * rowA);
        rsa[0] = make_rsrc(reinterpret_cast<const void *>(ptr[p0 + 1]), static_cast<uint32_t>(a.N * KB));
        ra[1] = DOWN ? ra[0] : make_rsrc(reinterpret_cast<const void *>(ptr[2]), static_cast<uint32_t>(a.N) * rowA);
        rsa[1] = DOWN ? rsa[0] : make_rsrc(reinterpret_cast<const void *>(ptr[3]), static_cast<uint32_t>(a.N * KB));
    }
    uint32_t aoff[4], asoff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = DOWN ? nt * 256 + wave * 64 + j * 16 + r16 : nt * 128 + wave * 32 + (j & 1) * 16 + r16;
        const bool ok = row < a.N;
        aoff[j] = ok ? static_cast<uint32_t>(row) * rowA + 32u * q : kOobOffset;
        asoff[j] = ok ? static_cast<uint32_t>(row * KB + 2 * q) : kOobOffset;
    }
    constexpr int kRing = 4;
    uint4 A[kRing][4][2];
    uint16_t SA[kRing][4];  // widened only where used, so no VALU op waits on the load early
    // Super-steps past the end load as zeros (block index >= KB), so every step issues the
    // same loads and the waits stay exact.  Invalid offsets keep bit 31 set (every valid
    // offset is below 2^31), OR-ed in without branches.
    auto load_a = [&](int S, int slot) {
        const uint32_t oob = S * 8 + 2 * q < KB ? 0u : kOobOffset;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t off = (aoff[j] + S * 128u) | oob;
            A[slot][j][0] = buf_load16(ra[j >> 1], off);
            A[slot][j][1] = buf_load16(ra[j >> 1], off + 16u);
            SA[slot][j] = __builtin_amdgcn_raw_buffer_load_b16(rsa[j >> 1], (asoff[j] + S * 8u) | oob, 0, 0);
        }
    };

    // ---- B staging.  Gate/up (x terms, gathered from memory): thread (column c = tid >> 4,
    // piece p = tid & 15) copies piece p of tile row c of every 16-column tile and term, so
    // one wave instruction reads four whole rows' 256-byte super-step runs (whole 128-byte
    // lines; the loads of 16 rows x 64 bytes they replace measured 5% slower), and the LDS
    // tile keeps [piece][column] order for the operand reads with the column XOR-ed by the
    // piece, so neither the stores nor the reads meet bank conflicts.  Down (act terms, just
    // written and in cache): thread (c = tid & 15, p = tid >> 4), plain order (the line-wise
    // form measured 3-7% slower there).  (c = tid & 15, block pair g = (tid >> 4) & 3, tile
    // tid >> 6) copies one scale pair per term.  Two register sets: loads run two super-steps
    // ahead of their LDS stores.
    constexpr bool kLines = !DOWN;
    const auto rb = make_rsrc(a.b8, a.b_term * TERMS);
    const auto rbs = make_rsrc(a.bs, a.bs_term * TERMS);
    const int dc = kLines ? tid >> 4 : tid & 15, dp = kLines ? tid & 15 : tid >> 4;
    // LDS unit (16 bytes) of piece pc of column c within one tile and term
    auto bunit = [](int pc, int c) { return pc * 16 + (kLines ? c ^ pc : c); };
    const int dp_bb = 4 * ((dp >> 2) & 1) + 2 * ((dp & 3) >> 1) + (dp >> 3);  // block of piece dp
    uint32_t boff[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
        const int rr = ct * 16 + dc;
        int brow = -1;
        if (rr < rows) brow = DOWN ? pos0 + rr : a.perm[pos0 + rr] / a.top_k;
        boff[ct] = brow >= 0 ? static_cast<uint32_t>(brow) * a.Kpad + dp * 16u : kOobOffset;
    }
    const int sc_c = tid & 15, sg = (tid >> 4) & 3, sct = tid >> 6;
    uint32_t bsoff;
    {
        const int rr = sct * 16 + sc_c;
        int brow = -1;
        if (rr < rows) brow = DOWN ? pos0 + rr : a.perm[pos0 + rr] / a.top_k;
        bsoff = brow >= 0 ? static_cast<uint32_t>(brow) * (a.Kpad >> 5) + 2u * sg : kOobOffset;
    }
    // gate/up stages bf16 x's two terms two super-steps ahead (gathered token rows); down,
    // whose act terms were written just before and sit in cache, and gate/up over fp32 x's
    // three terms, one step ahead, to stay in registers
    constexpr int XD = (DOWN || TERMS == 3) ? 1 : 2;
    uint4 XR[XD][4][TERMS];
    uint16_t XS[XD][TERMS];
    auto load_x = [&](int S, int xs) {
        const uint32_t poob = S >= 0 && S * 8 + dp_bb < KB ? 0u : kOobOffset;
        const uint32_t soob = S >= 0 && S * 8 + 2 * sg < KB ? 0u : kOobOffset;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
            for (int t = 0; t < TERMS; ++t)
                XR[xs][ct][t] = buf_load16(rb, (boff[ct] + t * a.b_term + S * kSS) | poob);
#pragma unroll
        for (int t = 0; t < TERMS; ++t)
            XS[xs][t] = __builtin_amdgcn_raw_buffer_load_b16(rbs, (bsoff + t * a.bs_term + S * 8u) | soob, 0, 0);
    };
    auto store_x = [&](int xs, int buf) {
        uint4 *xt = smem + buf * kXT;
        uint16_t *st = ssm + buf * kST;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
            for (int t = 0; t < TERMS; ++t) xt[(ct * TERMS + t) * 256 + bunit(dp, dc)] = XR[xs][ct][t];
#pragma unroll
        for (int t = 0; t < TERMS; ++t) st[((sct * TERMS + t) * 16 + sc_c) * 4 + sg] = XS[xs][t];
    };

    f32x4 acc[4][4];  // [A tile j][B tile ct]
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) acc[j][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

    // MFMAs of one super-step.  B fragments are read from LDS one 16-column tile ahead of
    // their MFMAs, two sets live; the scheduling fences keep the compiler from hoisting all
    // four tiles' fragments at once (which costs ~128 registers and forces reuse of
    // registers whose loads are still in flight).
    auto compute = [&](int slot, int buf) {
        const uint4 *xt = smem + buf * kXT;
        const uint16_t *st = ssm + buf * kST;
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            if (ct < nct) {
#pragma unroll
                for (int t = 0; t < TERMS; ++t) {
                    const uint4 *xb = xt + (ct * TERMS + t) * 256;
                    const uint32_t sb = st[((ct * TERMS + t) * 16 + r16) * 4 + q];
                    const uint4 b00 = xb[bunit(q, r16)], b01 = xb[bunit(4 + q, r16)];
                    const uint4 b10 = xb[bunit(8 + q, r16)], b11 = xb[bunit(12 + q, r16)];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[j][ct] = mfma_fp4_fp8<0>(A[slot][j][0], b00, b01, acc[j][ct], SA[slot][j], sb);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[j][ct] = mfma_fp4_fp8<1>(A[slot][j][1], b10, b11, acc[j][ct], SA[slot][j], sb);
                }
            }
        }
    };
    // Super-step S: MFMAs on LDS tile S % 2 and A slot S % 4; then A(S + 4) into the freed
    // slot, B(S + 1) from registers into the other LDS tile, B(S + 1 + XD) into the freed
    // registers.  The loop starts at S = -4 with the MFMAs skipped, so the pipeline fills
    // through the same instruction stream as the steady state (a separate prologue leaves
    // the loop entry with a different set of loads in flight, and the compiler's waits at the
    // loop head then cover the worse of the two).
    auto step = [&](int S, int slot, int par) {
        __syncthreads();  // tile S is stored and every wave is done with tile S - 1
        if (S >= 0) compute(slot, par);
        load_a(S + kRing, slot);
        store_x((par ^ 1) % XD, par ^ 1);
        load_x(S + 1 + XD, (par ^ 1) % XD);
    };
#pragma unroll
    for (int xs = 0; xs < XD; ++xs) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct)
#pragma unroll
            for (int t = 0; t < TERMS; ++t) XR[xs][ct][t] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int t = 0; t < TERMS; ++t) XS[xs][t] = 0;
    }
    // Unrolled over the four ring slots, so slot and LDS-tile indices are compile-time.
    static_assert(kRing == 4, "the loop below is unrolled over the four ring slots");
    for (int S = -kRing; S < NS; S += 4) {
        step(S, 0, 0);
        if (S + 1 < NS) step(S + 1, 1, 1);
        if (S + 2 < NS) step(S + 2, 2, 0);
        if (S + 3 < NS) step(S + 3, 3, 1);
    }

    // ---- epilogues (C: lane holds weight rows 4q + v of each A tile, column r16 of each B tile)
    if constexpr (DOWN) {
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const int rr = ct * 16 + r16;
            if (ct < nct && rr < rows) {
                const int pair = a.perm[pos0 + rr];
                float *yrow = a.ypair + static_cast<int64_t>(pair) * a.N;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int row = nt * 256 + wave * 64 + j * 16 + 4 * q;
                    if (row < a.N) *reinterpret_cast<float4 *>(yrow + row) = __builtin_bit_cast(float4, acc[j][ct]);
                }
            }
        }
    } else {
        const int ib = nt * 128 + wave * 32;  // the wave's intermediate block
        if (ib < a.N) {
            const int blk = ib >> 5;
            const uint32_t pbase = mxb_offset(blk, 0) + 4u * q;  // half 0; half 1 is 16 bytes on
#pragma unroll
            for (int ct = 0; ct < 4; ++ct) {
                if (ct < nct) {
                    const int rr = ct * 16 + r16;
                    const bool ok = rr < rows;
                    float v[2][4];
                    float amax = 0.f;
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            v[j][i] = act_fn(acc[j][ct][i], acc[j + 2][ct][i], a.act_kind, a.beta, a.lbeta);
                            amax = fmaxf(amax, fabsf(v[j][i]));
                        }
                    const uint32_t pos = static_cast<uint32_t>(pos0 + rr);
#pragma unroll
                    for (int tt = 0; tt < 3; ++tt) {
                        amax = fmaxf(amax, shfl_xor_f(amax, 16));
                        amax = fmaxf(amax, shfl_xor_f(amax, 32));
                        const int ex = block_exp(amax);
                        uint32_t c[2] = {0u, 0u};
                        amax = 0.f;
#pragma unroll
                        for (int j = 0; j < 2; ++j)
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                float qv;
                                c[j] |= e4m3_rne(ldexpf(v[j][i], -ex), qv) << (8 * i);
                                v[j][i] -= ldexpf(qv, ex);
                                amax = fmaxf(amax, fabsf(v[j][i]));
                            }
                        if (ok) {
                            uint8_t *dst = a.a8 + tt * a.a_term + pos * static_cast<uint32_t>(a.Ipad) + pbase;
                            *reinterpret_cast<uint32_t *>(dst) = c[0];
                            *reinterpret_cast<uint32_t *>(dst + 16) = c[1];
                            if (q == 0)
                                a.as[tt * a.as_term + pos * static_cast<uint32_t>(a.Ipad >> 5) + blk] =
                                    static_cast<uint8_t>(ex + 127);
                        }
                    }
                }
            }
        }
    }
}

// LDS of mx_gemm_kernel: two B tiles and their scale pairs
constexpr size_t mx_lds_bytes(int terms) {
    return 2 * (static_cast<size_t>(4 * terms * 16 * 16) * 16 + static_cast<size_t>(4 * terms * 16 * 4) * 2);
}

// Grid of mx_gemm_kernel: every (tile, row block) pair; tile major rounds the tiles up to a
// multiple of the 8 XCDs.
unsigned mx_grid(const MxArgs &m) {
    const int64_t tiles = m.tile_major ? 8 * cdiv(m.max_tiles, 8) : m.max_tiles;
    return static_cast<unsigned>(tiles * m.NT);
}

// Both GEMMs take more than the default 64 KB of dynamic LDS (gfx950 has 160 KB per CU).
int mx_prepare() {
    static const hipError_t rc = [] {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&mx_gemm_kernel<false, 2>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           static_cast<int>(mx_lds_bytes(2)));
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void *>(&mx_gemm_kernel<false, 3>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(mx_lds_bytes(3)));
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void *>(&mx_gemm_kernel<true, 3>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(mx_lds_bytes(3)));
        return e;
    }();
    return check_hip(rc, "moe grouped: LDS size attribute");
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
    size_t counts, base, perm, tile_e, tile_m0, n_tiles, x8, xs, a8, as, ypair, total;
    int max_tiles;
    int64_t Hpad, Ipad;
};

GroupedWs grouped_ws_layout(int64_t T, int64_t k, int64_t E, int64_t H, int64_t I) {
    GroupedWs L{};
    auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
    const int64_t P = T * k;
    L.Hpad = cdiv(H, kSS) * kSS;
    L.Ipad = cdiv(I, kSS) * kSS;
    L.max_tiles = static_cast<int>(cdiv(P, kTM) + E);
    size_t o = 0;
    L.counts = o, o += up(E * 4);
    L.base = o, o += up(E * 4);
    L.perm = o, o += up(P * 4);
    L.tile_e = o, o += up(static_cast<size_t>(L.max_tiles) * 4);
    L.tile_m0 = o, o += up(static_cast<size_t>(L.max_tiles) * 4);
    L.n_tiles = o, o += up(4);
    L.x8 = o, o += up(static_cast<size_t>(3) * T * L.Hpad);
    L.xs = o, o += up(static_cast<size_t>(3) * T * (L.Hpad / 32));
    L.a8 = o, o += up(static_cast<size_t>(3) * P * L.Ipad);
    L.as = o, o += up(static_cast<size_t>(3) * P * (L.Ipad / 32));
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
    if (x_dtype != K3_BF16 && x_dtype != K3_F32)
        return set_error(K3_ERR_DTYPE, "moe grouped: x must be bf16 or fp32 (x_dtype %d)", x_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "moe grouped: out_dtype");
    if (act_kind != K3_ACT_SILU && act_kind != K3_ACT_SITU) return set_error(K3_ERR_SHAPE, "moe grouped: act_kind");
    if (T <= 0 || top_k <= 0 || top_k > 64 || n_experts <= 0 || n_experts > 1024)
        return set_error(K3_ERR_SHAPE, "moe grouped: T >= 1, 1 <= top_k <= 64, 1 <= n_experts <= 1024 required");
    if (H <= 0 || I <= 0 || H % 64 || I % 64)
        return set_error(K3_ERR_SHAPE, "moe grouped: H=%lld and I=%lld must be positive multiples of 64",
                         (long long)H, (long long)I);
    const GroupedWs L = grouped_ws_layout(T, top_k, n_experts, H, I);
    const int64_t P = T * top_k;
    if (P >= (1ll << 30) || H * I / 2 >= (1ll << 31) || 3 * P * L.Ipad >= (1ll << 31) ||
        3 * T * L.Hpad >= (1ll << 31))
        return set_error(K3_ERR_SHAPE, "moe grouped: problem too large");
    if (workspace_bytes < static_cast<int64_t>(L.total))
        return set_error(K3_ERR_WORKSPACE, "moe grouped: workspace %lld < %zu bytes", (long long)workspace_bytes,
                         L.total);
    if (!aligned16(x) || !aligned16(workspace) || !aligned16(out))
        return set_error(K3_ERR_ALIGN, "moe grouped: x, out and workspace must be 16-byte aligned");
    auto st = static_cast<hipStream_t>(stream);
    char *ws = static_cast<char *>(workspace);

    GroupArgs g{};
    g.idx = expert_idx;
    g.P = static_cast<int>(P);
    g.E = static_cast<int>(n_experts);
    g.counts = reinterpret_cast<int32_t *>(ws + L.counts);
    g.base = reinterpret_cast<int32_t *>(ws + L.base);
    g.perm = reinterpret_cast<int32_t *>(ws + L.perm);
    g.tile_e = reinterpret_cast<int32_t *>(ws + L.tile_e);
    g.tile_m0 = reinterpret_cast<int32_t *>(ws + L.tile_m0);
    g.n_tiles = reinterpret_cast<int32_t *>(ws + L.n_tiles);
    g.max_tiles = L.max_tiles;
    group_count_kernel<<<dim3(g.E), kScanThreads, 0, st>>>(g);
    group_plan_kernel<<<dim3(1), 1024, 0, st>>>(g);
    group_place_kernel<<<dim3(g.E), kScanThreads, 0, st>>>(g);
    int rc = check_hip(hipGetLastError(), "moe grouped: grouping launches");
    if (rc) return rc;

    QxArgs qa{};
    qa.x = x;
    qa.x8 = reinterpret_cast<uint8_t *>(ws + L.x8);
    qa.xs = reinterpret_cast<uint8_t *>(ws + L.xs);
    qa.T = static_cast<int>(T);
    qa.H = static_cast<int>(H);
    qa.Hpad = static_cast<int>(L.Hpad);
    qa.term = static_cast<uint32_t>(T * L.Hpad);
    qa.sterm = static_cast<uint32_t>(T * (L.Hpad / 32));
    const bool xf32 = x_dtype == K3_F32;
    if (xf32)
        quant_x_kernel<true><<<dim3(static_cast<unsigned>(cdiv(T * (H / 16), 256))), 256, 0, st>>>(qa);
    else
        quant_x_kernel<false><<<dim3(static_cast<unsigned>(cdiv(T * (H / 16), 256))), 256, 0, st>>>(qa);
    rc = check_hip(hipGetLastError(), "moe grouped: x quantization launch");
    if (rc) return rc;

    rc = mx_prepare();
    if (rc) return rc;
    MxArgs ma{};
    ma.table = static_cast<const uint64_t *>(expert_table);
    ma.counts = g.counts;
    ma.base = g.base;
    ma.perm = g.perm;
    ma.tile_e = g.tile_e;
    ma.tile_m0 = g.tile_m0;
    ma.n_tiles = g.n_tiles;
    ma.a8 = reinterpret_cast<uint8_t *>(ws + L.a8);
    ma.as = reinterpret_cast<uint8_t *>(ws + L.as);
    ma.a_term = static_cast<uint32_t>(P * L.Ipad);
    ma.as_term = static_cast<uint32_t>(P * (L.Ipad / 32));
    ma.Ipad = static_cast<int>(L.Ipad);
    ma.ypair = reinterpret_cast<float *>(ws + L.ypair);
    ma.top_k = static_cast<int>(top_k);
    ma.max_tiles = L.max_tiles;
    ma.act_kind = act_kind;
    ma.beta = beta;
    ma.lbeta = linear_beta;
    // gate/up: K = H, weight rows N = I, 128 intermediate indices per block
    ma.b8 = qa.x8;
    ma.bs = qa.xs;
    ma.b_term = qa.term;
    ma.bs_term = qa.sterm;
    ma.K = static_cast<int>(H);
    ma.Kpad = static_cast<int>(L.Hpad);
    ma.N = static_cast<int>(I);
    ma.NT = static_cast<int>(cdiv(I, 128));
    ma.tile_major = 0;
    const dim3 gu_grid(mx_grid(ma));
    if (xf32)
        mx_gemm_kernel<false, 3><<<gu_grid, kThreads, mx_lds_bytes(3), st>>>(ma);
    else
        mx_gemm_kernel<false, 2><<<gu_grid, kThreads, mx_lds_bytes(2), st>>>(ma);
    rc = check_hip(hipGetLastError(), "moe grouped: gate/up launch");
    if (rc) return rc;
    // down: K = I, weight rows N = H, 256 output rows per block, B = the act terms
    ma.b8 = ma.a8;
    ma.bs = ma.as;
    ma.b_term = ma.a_term;
    ma.bs_term = ma.as_term;
    ma.K = static_cast<int>(I);
    ma.Kpad = static_cast<int>(L.Ipad);
    ma.N = static_cast<int>(H);
    ma.NT = static_cast<int>(cdiv(H, 256));
    ma.tile_major = 1;
    mx_gemm_kernel<true, 3><<<dim3(mx_grid(ma)), kThreads, mx_lds_bytes(3), st>>>(ma);
    rc = check_hip(hipGetLastError(), "moe grouped: down launch");
    if (rc) return rc;

    CombineArgs ca{ma.ypair, expert_w, out, static_cast<int>(T), static_cast<int>(H), static_cast<int>(top_k),
                   out_dtype == K3_BF16};
    combine_kernel<<<dim3(static_cast<unsigned>(T), static_cast<unsigned>(cdiv(H, 1024))), 256, 0, st>>>(ca);
    return check_hip(hipGetLastError(), "moe grouped: combine launch");
}
