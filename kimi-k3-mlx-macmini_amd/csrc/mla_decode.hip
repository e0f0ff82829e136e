// Latent-MLA absorbed decode attention for one query token (batch 1) over a bf16
// compressed cache, on gfx950.
//
// Reference: MLAAttention.__call__ (air_llm/models/kimi_k3/attention_mla.py:193-212), for
// T == 1 (no causal mask, attention_mla.py:200-207):
//     qa  = q_nope @ W_UK                 [H, r]
//     s   = (qa . lat^T + q_rot . rot^T) * scale
//     p   = softmax_fp32(s)
//     ctx = p @ lat                       [H, r]
//     o   = ctx @ W_UV^T                  [H, v]
// The reference upcasts the whole cache prefix to fp32 every step (attention_mla.py:85-87).
// Here the cache stays bf16 and is read once; four stream-ordered launches:
//
//   Q   qa[h] = q_nope[h] @ W_UK[h] in fp32, stored as a bf16 hi/lo pair
//       (hi = rne(qa), lo = rne(qa - hi)), together with q_rot in columns 512..575, so the
//       score contraction is one K = 576 product against the [lat | rot] cache rows.
//   A   split-T flash decoding.  A block owns 16 heads and a contiguous token range (one
//       block per CU, eight waves).  Cache rows arrive as whole 1 KB rows per load
//       instruction into an LDS ring; four score waves take S^T[16 tokens x 16 heads] as bf16
//       MFMAs (v_mfma_f32_16x16x32_bf16) of the rows against the hi and the lo half of qa,
//       in K halves that meet through LDS, and a base-2 softmax turns them into P, split
//       again into a bf16 hi/lo pair; four context waves take ctx^T += rows^T [P_hi; P_lo]
//       on the same MFMA from transposed LDS reads.  The two tile classes merge in the
//       block, which writes its unnormalised (ctx, max, sum) record per head.
//   M   per (head, quarter of the latent columns): log-sum-exp merge of the split records
//       in a fixed order into the normalised ctx, then the W_UV product over that quarter,
//       o_q = W_UV[h][:, quarter] @ ctx[h][quarter] in fp32; every record and W_UV element is
//       read by one block.
//   O   o = o_0 + o_1 + o_2 + o_3 in quarter order (then the optional output gate).
//
// Numerics: lat, rot, W_UK, W_UV and bf16 queries are exact in the MFMA inputs; the fp32
// operands (qa, P) are carried as hi + lo bf16 pairs, so each product is represented to
// ~2^-17 relative before fp32 accumulation -- fp32-class results from bf16 matrix cores.
#include <algorithm>

#include "k3_common.h"

namespace k3 {
namespace {

constexpr int kR = 512;          // kv_lora_rank (latent width)
constexpr int kRope = 64;        // rope key width
constexpr int kK = kR + kRope;   // score contraction length
constexpr int kQaLd = kK;        // row stride of the qa hi/lo arrays in the workspace
constexpr int kHG = 16;          // heads per attention block (one MFMA tile)
constexpr int kMaxSplits = 1024;
constexpr int kKSteps = kK / 32; // 18 MFMA k-steps over the score contraction

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma_bf16(bf16x8 a, bf16x8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Reductions over the 16 lanes of a DPP row (lanes 16r .. 16r+15), result in every lane of
// the row: quad swaps, then half-row and row mirrors.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, dpp_move<0xb1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_move<0x4e>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_move<0x141>(v));  // row_half_mirror
    return fmaxf(v, dpp_move<0x140>(v));  // row_mirror
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_move<0xb1>(v);
    v += dpp_move<0x4e>(v);
    v += dpp_move<0x141>(v);
    return v + dpp_move<0x140>(v);
}

// fp32 -> (hi, lo) bf16 bit patterns with hi + lo == v to ~2^-17 relative
__device__ __forceinline__ void split_bf16(float v, uint16_t &hi, uint16_t &lo) {
    hi = f32_to_bf16(v);
    lo = f32_to_bf16(v - bf16_to_f32(hi));
}

template <typename QT>
__device__ __forceinline__ float load_q(const QT *p) {
    if constexpr (std::is_same<QT, float>::value)
        return *p;
    else
        return bf16_to_f32(*p);
}

// ------------------------------------------------------------------ Q: qa = q_nope @ W_UK
struct QaArgs {
    const void *q_nope, *q_rot;  // [H, ld_q] and [H, ld_q_rot] rows (bf16 or fp32)
    int64_t ld_q, ld_q_rot;
    const uint16_t *w_uk;        // [H, nope, 512] bf16
    uint16_t *qa_hi, *qa_lo;     // [H, 576]
    int H, nope;
};

// grid: H * 4 blocks, block (h, quarter) produces qa[h][128*quarter .. +128)
template <typename QT>
__global__ __launch_bounds__(256) void mla_qa_kernel(QaArgs a) {
    __shared__ float qn[256];
    __shared__ float red[16][129];
    const int h = blockIdx.x >> 2, quarter = blockIdx.x & 3;
    const int tid = threadIdx.x;
    const QT *q = static_cast<const QT *>(a.q_nope) + static_cast<int64_t>(h) * a.ld_q;
    for (int n = tid; n < a.nope; n += 256) qn[n] = load_q(q + n);
    __syncthreads();
    const int rc = tid & 15, ng = tid >> 4;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const uint16_t *wrow = a.w_uk + static_cast<int64_t>(h) * a.nope * kR + quarter * 128 + rc * 8;
    uint4 wv[16];  // nope <= 256: every load of this thread in flight at once
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int n = ng + 16 * u;
        wv[u] = n < a.nope ? *reinterpret_cast<const uint4 *>(wrow + static_cast<int64_t>(n) * kR)
                           : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        const int n = ng + 16 * u;
        const float qv = n < a.nope ? qn[n] : 0.f;
        const uint32_t wd[4] = {wv[u].x, wv[u].y, wv[u].z, wv[u].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[2 * j] = fmaf(qv, __uint_as_float(wd[j] << 16), acc[2 * j]);
            acc[2 * j + 1] = fmaf(qv, __uint_as_float(wd[j] & 0xffff0000u), acc[2 * j + 1]);
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) red[ng][rc * 8 + j] = acc[j];
    __syncthreads();
    if (tid < 128) {
        float v = 0.f;
        for (int g = 0; g < 16; ++g) v += red[g][tid];
        uint16_t hi, lo;
        split_bf16(v, hi, lo);
        a.qa_hi[h * kQaLd + quarter * 128 + tid] = hi;
        a.qa_lo[h * kQaLd + quarter * 128 + tid] = lo;
    } else if (quarter == 0 && tid < 128 + kRope) {
        const int j = tid - 128;
        const float v = load_q(static_cast<const QT *>(a.q_rot) + static_cast<int64_t>(h) * a.ld_q_rot + j);
        uint16_t hi, lo;
        split_bf16(v, hi, lo);
        a.qa_hi[h * kQaLd + kR + j] = hi;
        a.qa_lo[h * kQaLd + kR + j] = lo;
    }
}

// ------------------------------------------------------------------ A: split-T attention
struct AttnArgs {
    const uint16_t *qa_hi, *qa_lo;  // [H, 576]
    const void *lat;                // [T, ld_lat] bf16
    const void *rot;                // [T, ld_rot] bf16
    uint32_t lat_bytes, rot_bytes;  // readable bytes from each base
    uint32_t lat_row_bytes, rot_row_bytes;  // bytes between tokens
    float *part;                    // [NS, H, 512] unnormalised context per split and head
    float2 *ml;                     // [NS, H] (running max, running sum) per split and head
    int H, T, Ts, NS;
    float scale_log2;               // softmax scale * log2(e)
    int swizzle;                    // XCD-aware block -> work mapping
};

// Sum / max over the four 16-lane rows of the wave (lanes l, l^16, l^32, l^48), result in
// every lane; the row pairs are combined in a fixed order, so the sum is deterministic.
__device__ __forceinline__ float rows4_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float rows4_max(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// bf16 pair (RNE, hardware conversion) of (a, b): low half a
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
    return __builtin_bit_cast(uint32_t, v);
}

typedef short s4_t __attribute__((ext_vector_type(4)));

// Block: 16 heads x one split of Ts tokens, eight waves (two per SIMD) in two roles.  The
// split is walked in rounds of two 16-token tiles; tile c of a round belongs to tile class c.
//   staging (all waves): the round's latent rows arrive one whole 1 KB row per load
//           instruction (whole 128-byte lines), through registers (D rounds in flight) into
//           an LDS ring of four rounds, rows padded (kLatStride) for the operand reads.
//   score waves (0..3), class c = w / 2, half h = w % 2: the partial S^T[token][head] of tile
//           c over latent columns 256 h .. +256 and rope columns 32 h .. +32, on 16x16x32 bf16
//           MFMAs (A = the staged rows read with ds_read_b128, rope rows loaded directly in
//           operand layout; B = qa hi and lo for those columns, in registers for the whole
//           split), four accumulator chains.  The two halves' partials meet through LDS; both
//           waves add them in the same order, so both hold identical scores.  Lane (head r16,
//           q4) holds tokens 4 q4 .. +3.  Softmax per lane over its 4 tokens, the max reduced
//           over the 4 lane rows; each head keeps a reference max per class: exponentials
//           are 2^(s - ref) <= 2^kSlack, and a score above the reference by more than kSlack
//           (log2 units) moves it, with the factor 2^(old - new) for the accumulators.  P
//           (hi/lo bf16, in the B-operand layout) and the factors go to LDS.
//   context waves (4..7), class c, half h: ctx^T[col][head] += rows^T . [P_hi; P_lo] over
//           latent columns 256 h .. +256 of tile c on the 16x16x32 MFMA, k-slots 0..3 = P_hi
//           and 4..7 = P_lo of the lane's own 4 tokens; the transposed rows come from the
//           staged tile (ds_read_b64_tr_b16), duplicated into both k halves.
// One barrier per round: in iteration r the score waves finish round r's softmax and start
// round r + 1's partial scores, while the context waves take round r - 1's products.  At the
// end the two classes merge (common reference, fixed order) and the block writes its
// unnormalised context per head and (reference max, sum) for the merge kernel.
constexpr int kStepT = 16;                          // tokens per tile
constexpr int kLatStride = 1056;                    // LDS bytes per staged latent row (1024 + 32)
constexpr int kTileLds = kStepT * kLatStride;       // 16896 B per staged tile
constexpr int kRoundTiles = 2;                      // tiles per round (tile classes)
constexpr int kRoundLds = kRoundTiles * kTileLds;
constexpr int kSlots = 4;                           // staged rounds in LDS
constexpr int kChunks = kRoundTiles * kStepT;       // 1 KB row loads per round
constexpr int kPerWave = (kChunks + 7) / 8;         // row loads per wave and round
constexpr int kHalfKb = kR / 64;                    // latent k-blocks (of 32) per score half: 8
constexpr int kColTiles = kR / 2 / 16;              // context column tiles per context wave: 16
constexpr float kSlack = 64.f;                      // log2 headroom before a reference moves
constexpr size_t kAttnLds = static_cast<size_t>(kSlots) * kRoundLds;  // 135168 B
static_assert(static_cast<size_t>(kHG) * kR * 4 <= kAttnLds, "class merge staging fits");

// F32: the cache holds fp32 rows (the reference's default cache dtype).  A round is then one
// 16-token tile staged as two bf16 planes, hi = rne(v) and lo = rne(v - hi), and the tile
// classes become the planes: class 0 works on the hi plane, class 1 on the lo plane of the
// same tokens.  The score waves' partials of both planes add into one score (so both classes
// run the same softmax, with identical references and sums), and each class's context waves
// take plane^T . [P_hi; P_lo]; the two contexts add at the end.  Every product of
// (hi + lo) x (hi + lo) is kept, so the fp32 rows enter to ~2^-16 relative.
template <int D, bool F32>
__global__ __launch_bounds__(512, 1) void mla_attn_kernel(AttnArgs a) {
    static_assert(D >= 2, "rounds 0 and 1 are staged from two register slots");
    constexpr int kRoundTok = F32 ? kStepT : kStepT * kRoundTiles;  // tokens per round
    constexpr int RP = F32 ? 2 : 1;                                 // 16-byte rope loads per lane
    extern __shared__ uint4 smem[];
    __shared__ f32x4_t xs[2][kRoundTiles][2][64];   // partial scores [parity][class][half][lane]
    __shared__ uint4 xp[2][kRoundTiles][64];        // P hi/lo [parity][class][lane]
    __shared__ float xf[2][kRoundTiles][kHG];       // rescale factors [parity][class][head]
    __shared__ float2 xm[kRoundTiles][kHG];         // final (reference, sum) [class][head]
    char *lds = reinterpret_cast<char *>(smem);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool ctx_role = wave >= 4;
    const int cls = (wave & 3) >> 1, half = wave & 1;
    const int r16 = lane & 15, q4 = lane >> 4;

    // blocks b, b+8, b+16, ... share an XCD (and its L2): give them consecutive work items,
    // so the head groups of one split read the same rows through one L2
    const int b = blockIdx.x;
    const int w = a.swizzle ? (b & 7) * (static_cast<int>(gridDim.x) >> 3) + (b >> 3) : b;
    const int HGn = (a.H + kHG - 1) / kHG;
    const int hg = w % HGn, split = w / HGn;
    const int h0 = hg * kHG;
    const int t_begin = split * a.Ts;
    const int t_end = min(a.T, t_begin + a.Ts);
    const int nsteps = (t_end - t_begin + kStepT - 1) / kStepT;   // tiles of the split
    const int nrounds = F32 ? nsteps : (nsteps + kRoundTiles - 1) / kRoundTiles;
    // the 16-token tile that class c works on in round rd
    auto tile_of = [&](int rd, int c) { return F32 ? rd : rd * kRoundTiles + c; };
    const int nloop = (nrounds + 1 + D - 1) / D * D;              // one more for the context waves
    auto slot = [&](int rd) { return lds + (rd % kSlots) * kRoundLds; };

    // ---- staging, all eight waves: row load q = wave + 8 i of a round (tile q / 16, row
    // q % 16); tiles and rows past the split load zeros (out-of-range offsets), so every
    // round issues the same loads
    const auto rl = make_rsrc(a.lat, a.lat_bytes);
    // bf16: load q is row q % 16 of tile 2 rd + q / 16, whole (1 KB);  fp32: load q is half
    // q % 2 (1 KB, 256 values) of row q / 2 of tile rd
    auto load_round = [&](uint4 (&g)[kPerWave], int rd) {
#pragma unroll
        for (int i = 0; i < kPerWave; ++i) {
            const int q = wave + 8 * i;
            const int tile = F32 ? rd : rd * kRoundTiles + q / kStepT;
            const int row = F32 ? q / 2 : q % kStepT;
            const int t = t_begin + tile * kStepT + row;
            const bool ok = q < kChunks && tile < nsteps && t < t_end;
            const uint32_t col = F32 ? (q % 2) * 1024u + lane * 16u : lane * 16u;
            g[i] = buf_load16(rl, ok ? static_cast<uint32_t>(t) * a.lat_row_bytes + col : kOobOffset);
        }
    };
    auto store_round = [&](const uint4 (&g)[kPerWave], int rd) {
        char *base = slot(rd);
#pragma unroll
        for (int i = 0; i < kPerWave; ++i) {
            const int q = wave + 8 * i;
            if (q < kChunks) {
                if constexpr (F32) {
                    // four fp32 values -> their hi bf16 (plane 0) and lo bf16 (plane 1)
                    const float v0 = __uint_as_float(g[i].x), v1 = __uint_as_float(g[i].y);
                    const float v2 = __uint_as_float(g[i].z), v3 = __uint_as_float(g[i].w);
                    const uint32_t h01 = pack_bf16x2(v0, v1), h23 = pack_bf16x2(v2, v3);
                    const uint32_t l01 = pack_bf16x2(v0 - __uint_as_float(h01 << 16), v1 - __uint_as_float(h01 & 0xffff0000u));
                    const uint32_t l23 = pack_bf16x2(v2 - __uint_as_float(h23 << 16), v3 - __uint_as_float(h23 & 0xffff0000u));
                    char *row = base + (q / 2) * kLatStride + ((q % 2) * 256 + lane * 4) * 2;
                    *reinterpret_cast<uint2 *>(row) = make_uint2(h01, h23);
                    *reinterpret_cast<uint2 *>(row + kTileLds) = make_uint2(l01, l23);
                } else {
                    *reinterpret_cast<uint4 *>(base + (q / kStepT) * kTileLds + (q % kStepT) * kLatStride + lane * 16) =
                        g[i];
                }
            }
        }
    };
    uint4 stg[D][kPerWave];
    load_round(stg[0], 0);
    load_round(stg[1], 1);
    // score waves: qa operands (head h0 + r16, this half's columns; heads past H load zeros)
    // and the first rounds' rope rows, issued together with the first rounds' latent rows so
    // their latencies overlap (context waves issue none of them)
    bf16x8 qhi[kHalfKb + 1], qlo[kHalfKb + 1];
    const auto rr = make_rsrc(a.rot, a.rot_bytes);
    // the 8 rope values (columns 32 half + 8 q4 ..) of token r16 of the class's tile: one
    // 16-byte load of bf16 rows, two of fp32 rows (split into the class's plane at use)
    typedef uint4 RopeRaw[RP];
    auto load_rope = [&](RopeRaw &o, int rd) {
        const int tile = tile_of(rd, cls);
        const int t = t_begin + tile * kStepT + r16;
        const bool ok = tile < nsteps && t < t_end;
        const uint32_t off = static_cast<uint32_t>(t) * a.rot_row_bytes + (half * 32 + q4 * 8) * (F32 ? 4u : 2u);
#pragma unroll
        for (int j = 0; j < RP; ++j) o[j] = buf_load16(rr, ok ? off + 16u * j : kOobOffset);
    };
    RopeRaw rope[D], rope0;
    if (!ctx_role) {
        const uint32_t qbytes = static_cast<uint32_t>(a.H) * kQaLd * 2;
        const auto rqh = make_rsrc(a.qa_hi, qbytes), rql = make_rsrc(a.qa_lo, qbytes);
        const uint32_t qrow = h0 + r16 < a.H ? static_cast<uint32_t>((h0 + r16) * kQaLd) * 2u : kOobOffset;
#pragma unroll
        for (int k = 0; k <= kHalfKb; ++k) {
            const int col = k < kHalfKb ? (half * kHalfKb + k) * 32 + q4 * 8 : kR + half * 32 + q4 * 8;
            qhi[k] = __builtin_bit_cast(bf16x8, buf_load16(rqh, qrow + static_cast<uint32_t>(col) * 2u));
            qlo[k] = __builtin_bit_cast(bf16x8, buf_load16(rql, qrow + static_cast<uint32_t>(col) * 2u));
        }
#pragma unroll
        for (int d = 1; d <= D; ++d) load_rope(rope[d % D], d);
        load_rope(rope0, 0);
    }
    store_round(stg[0], 0);
    store_round(stg[1], 1);
#pragma unroll
    for (int d = 0; d < D; ++d) load_round(stg[(2 + d) % D], 2 + d);

    float *cs = reinterpret_cast<float *>(lds);  // class 1's scaled context at the end, [16][kR]
    typedef __attribute__((address_space(3))) s4_t *lds_s4;

    if (!ctx_role) {
        // ================= score waves
        float m_ref = -INFINITY, l_run = 0.f;  // head h0 + r16, class cls (both halves alike)
        // partial scores of round rd over this half's columns
        auto partial = [&](int rd, const RopeRaw &rp) -> f32x4_t {
            const char *arow = slot(rd) + cls * kTileLds + r16 * kLatStride + half * 512 + q4 * 16;
            auto rdk = [&](int k) { return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(arow + k * 64)); };
            f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0, s2 = s0, s3 = s0;
            bf16x8 c[kHalfKb];
#pragma unroll
            for (int k = 0; k < 4; ++k) c[k] = rdk(k);
#pragma unroll
            for (int k = 0; k < kHalfKb; k += 2) {
                if (k + 4 < kHalfKb) {
                    c[k + 4] = rdk(k + 4);
                    c[k + 5] = rdk(k + 5);
                }
                s0 = mfma_bf16(c[k], qhi[k], s0);
                s1 = mfma_bf16(c[k], qlo[k], s1);
                s2 = mfma_bf16(c[k + 1], qhi[k + 1], s2);
                s3 = mfma_bf16(c[k + 1], qlo[k + 1], s3);
                __builtin_amdgcn_sched_barrier(0);
            }
            bf16x8 rk;
            if constexpr (F32) {
                // the class's plane of the 8 fp32 rope values: hi for class 0, lo for class 1
                const uint32_t v[8] = {rp[0].x, rp[0].y, rp[0].z, rp[0].w, rp[1].x, rp[1].y, rp[1].z, rp[1].w};
                uint32_t pk[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float f0 = __uint_as_float(v[2 * j]), f1 = __uint_as_float(v[2 * j + 1]);
                    const uint32_t hi = pack_bf16x2(f0, f1);
                    pk[j] = cls == 0 ? hi
                                     : pack_bf16x2(f0 - __uint_as_float(hi << 16), f1 - __uint_as_float(hi & 0xffff0000u));
                }
                rk = __builtin_bit_cast(bf16x8, make_uint4(pk[0], pk[1], pk[2], pk[3]));
            } else {
                rk = __builtin_bit_cast(bf16x8, rp[0]);
            }
            s0 = mfma_bf16(rk, qhi[kHalfKb], s0);
            s1 = mfma_bf16(rk, qlo[kHalfKb], s1);
            return (s0 + s2) + (s1 + s3);
        };
        // softmax of round rd from the two halves' partials; half 0 publishes P and factors
        auto softmax = [&](int rd) {
            // fp32 rows: the hi and lo planes' partials, in one order for both classes
            const f32x4_t sc = F32 ? (xs[rd & 1][0][0][lane] + xs[rd & 1][0][1][lane]) +
                                         (xs[rd & 1][1][0][lane] + xs[rd & 1][1][1][lane])
                                   : xs[rd & 1][cls][0][lane] + xs[rd & 1][cls][1][lane];
            const int tbeg = t_begin + tile_of(rd, cls) * kStepT + q4 * 4;
            float sv[4];
            float mt = -INFINITY;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                sv[v] = tbeg + v < t_end ? sc[v] * a.scale_log2 : -INFINITY;
                mt = fmaxf(mt, sv[v]);
            }
            mt = rows4_max(mt);  // this head's max over the tile; -inf for a fully masked tile
            float f = 1.f;
            if (__any(mt > m_ref + kSlack)) {
                const float m_new = mt > m_ref + kSlack ? mt : m_ref;
                if (m_new != m_ref) {
                    f = m_ref == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_ref - m_new);
                    l_run *= f;
                    m_ref = m_new;
                }
            }
            // p <= 2^kSlack; exponents below -126 flush to 0, far below the head's largest p.
            // Before the class's first token of the head the reference is -inf and every p is 0.
            const float mref = m_ref == -INFINITY ? 0.f : m_ref;
            uint32_t pw[4];
#pragma unroll
            for (int v = 0; v < 4; v += 2) {
                const float p0 = __builtin_amdgcn_exp2f(sv[v] - mref), p1 = __builtin_amdgcn_exp2f(sv[v + 1] - mref);
                l_run += p0 + p1;
                const uint32_t hi = pack_bf16x2(p0, p1);
                pw[v / 2] = hi;
                pw[2 + v / 2] = pack_bf16x2(p0 - __uint_as_float(hi << 16), p1 - __uint_as_float(hi & 0xffff0000u));
            }
            if (half == 0) {
                xp[rd & 1][cls][lane] = make_uint4(pw[0], pw[1], pw[2], pw[3]);
                if (q4 == 0) xf[rd & 1][cls][r16] = f;
            }
        };
        __syncthreads();  // rounds 0 and 1 staged
        xs[0][cls][half][lane] = partial(0, rope0);
        __syncthreads();  // partials of round 0 published
        for (int r0 = 0; r0 < nloop; r0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const int rd = r0 + d;
                store_round(stg[(d + 2) % D], rd + 2);
                load_round(stg[(d + 2) % D], rd + 2 + D);
                // round rd + 1's rope sits in rope[(rd + 1) % D] (r0 is a multiple of D)
                const int rs = (d + 1) % D;
                const f32x4_t pnext = partial(rd + 1, rope[rs]);
                softmax(rd);
                xs[(rd + 1) & 1][cls][half][lane] = pnext;
                load_rope(rope[rs], rd + 1 + D);
                __syncthreads();
            }
        }
        // (reference, sum) per class and head; wave 0 merges the classes and writes them
        const float l_tot = rows4_sum(l_run);
        if (half == 0 && q4 == 0) xm[cls][r16] = make_float2(m_ref, l_tot);
        __syncthreads();  // xm complete
        if (wave == 0 && q4 == 0 && h0 + r16 < a.H) {
            const float2 v = xm[0][r16], o = xm[1][r16];
            const float M = fmaxf(v.x, o.x);
            const float f0 = v.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(v.x - M);
            const float f1 = o.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(o.x - M);
            // fp32 rows: both classes summed the same tokens' probabilities (identically)
            a.ml[static_cast<int64_t>(split) * a.H + h0 + r16] = make_float2(M, F32 ? v.y : v.y * f0 + o.y * f1);
        }
        __syncthreads();  // class 1's context staged
    } else {
        // ================= context waves
        f32x4_t cacc[kColTiles];
#pragma unroll
        for (int n = 0; n < kColTiles; ++n) cacc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        __syncthreads();  // rounds 0 and 1 staged
        __syncthreads();  // partials of round 0 published
        for (int r0 = 0; r0 < nloop; r0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const int rd = r0 + d;
                store_round(stg[(d + 2) % D], rd + 2);
                load_round(stg[(d + 2) % D], rd + 2 + D);
                if (rd >= 1) {
                    // P and factors of round rd - 1 (published in the previous iteration)
                    const int pr = (rd - 1) & 1;
                    const bf16x8 pb = __builtin_bit_cast(bf16x8, xp[pr][cls][lane]);
                    const float fj = xf[pr][cls][r16];
                    if (__any(fj != 1.f)) {
#pragma unroll
                        for (int n = 0; n < kColTiles; ++n) cacc[n] *= fj;
                    }
                    const char *tsrc = slot(rd - 1) + cls * kTileLds + (q4 * 4 + (r16 >> 2)) * kLatStride +
                                       (half * (kR / 2) + (r16 & 3) * 4) * 2;
                    constexpr int kTrAhead = 8;  // transposed reads in flight ahead of the products
                    s4_t t4[kTrAhead];
#pragma unroll
                    for (int n = 0; n < kTrAhead; ++n)
                        t4[n] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(tsrc + n * 32));
#pragma unroll
                    for (int n = 0; n < kColTiles; ++n) {
                        const s4_t cur = t4[n % kTrAhead];
                        if (n + kTrAhead < kColTiles)
                            t4[n % kTrAhead] =
                                __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(tsrc + (n + kTrAhead) * 32));
                        const bf16x8 ra =
                            __builtin_bit_cast(bf16x8, __builtin_shufflevector(cur, cur, 0, 1, 2, 3, 0, 1, 2, 3));
                        cacc[n] = mfma_bf16(ra, pb, cacc[n]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                __syncthreads();
            }
        }
        __syncthreads();  // xm complete; every wave is done with the staged tiles
        const float mc = xm[cls][r16].x, mo = xm[1 - cls][r16].x;
        const float M = fmaxf(mc, mo);  // -inf only if neither class saw a token
        const float fc = mc == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mc - M);
        float *crow = cs + r16 * kR + half * (kR / 2) + 4 * q4;
        if (cls == 1) {
#pragma unroll
            for (int n = 0; n < kColTiles; ++n) *reinterpret_cast<f32x4_t *>(crow + 16 * n) = cacc[n] * fc;
        }
        __syncthreads();  // class 1's context staged
        if (cls == 0 && h0 + r16 < a.H) {
            float *rec = a.part + (static_cast<int64_t>(split) * a.H + h0 + r16) * kR + half * (kR / 2) + 4 * q4;
#pragma unroll
            for (int n = 0; n < kColTiles; ++n)
                *reinterpret_cast<f32x4_t *>(rec + 16 * n) =
                    cacc[n] * fc + *reinterpret_cast<const f32x4_t *>(crow + 16 * n);
        }
    }
}

// ------------------------------------------------------------------ M: merge, then W_UV
struct MergeArgs {
    const float *part;     // [NS, H, 512]
    const float2 *ml;      // [NS, H]
    const uint16_t *w_uv;  // [H, V, 512] bf16
    float *opart;          // [4, H, V] W_UV products over each quarter of the columns
    int H, NS, V;
};

__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = wave_sum_all(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return r;
}
__device__ __forceinline__ float block_max256(float v, float *red) {
    v = wave_max_all(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float r = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    return r;
}

constexpr int kMergeQ = 4;                   // column quarters per head
constexpr int kMQCols = kR / kMergeQ;        // 128 columns per merge block
constexpr int kMergeChunk = 16;              // record loads per thread in flight at once
constexpr int kUvBatch = 8;                  // W_UV row groups (16 rows) in flight at once

// grid: H * 4; block (h, q) owns columns 128 q .. +128 of head h.  Each record column is read
// by exactly one block, and so is each W_UV element.
//   merge:  ctx = sum_s 2^(m_s - M) ctx_s / L with M = max_s m_s, L = sum_s 2^(m_s - M) l_s;
//           thread t owns columns 4 (t % 32) .. +3 of the splits s = t / 32 (mod 8), the eight
//           partial sums meet in LDS and add in split-group order
//   W_UV:   opart[q][h][v] = W_UV[h][v][128 q ..] . ctx; 16 lanes per row (8 columns each),
//           so one wave instruction reads four whole 256-byte row pieces
__global__ __launch_bounds__(256) void mla_merge_kernel(MergeArgs a) {
    __shared__ float4 red8[8][kMQCols / 4];
    __shared__ float ctx[kMQCols];
    __shared__ float wsplit[kMaxSplits];
    __shared__ float red[4];
    const int h = blockIdx.x / kMergeQ, q = blockIdx.x % kMergeQ;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c4 = tid & 31, g = tid >> 5;
    const int sub = lane & 15;  // W_UV: lane covers columns 8 sub .. +8 of the quarter

    // first batch of W_UV rows: wave w, rows 16 i + 4 w + lane / 16
    const uint16_t *wbase = a.w_uv + static_cast<int64_t>(h) * a.V * kR + q * kMQCols + sub * 8;
    auto w_row = [&](int v) -> uint4 {
        return v < a.V ? *reinterpret_cast<const uint4 *>(wbase + static_cast<int64_t>(v) * kR) : make_uint4(0u, 0u, 0u, 0u);
    };
    const int vrow = 4 * wave + (lane >> 4);
    uint4 w[kUvBatch];
#pragma unroll
    for (int i = 0; i < kUvBatch; ++i) w[i] = w_row(16 * i + vrow);
    // split maxima and sums
    float2 mlv[kMaxSplits / 256];
#pragma unroll
    for (int u = 0; u < kMaxSplits / 256; ++u) {
        const int sidx = tid + 256 * u;
        mlv[u] = sidx < a.NS ? a.ml[static_cast<int64_t>(sidx) * a.H + h] : make_float2(-INFINITY, 0.f);
    }
    // record columns of the first chunk of splits
    const float *col = a.part + static_cast<int64_t>(h) * kR + q * kMQCols + 4 * c4;
    const int64_t sstride = static_cast<int64_t>(a.H) * kR;
    auto load_chunk = [&](float4(&c)[kMergeChunk], int s0) {
#pragma unroll
        for (int u = 0; u < kMergeChunk; ++u) {
            const int sidx = s0 + 8 * u + g;
            c[u] = sidx < a.NS ? *reinterpret_cast<const float4 *>(col + sidx * sstride) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    float4 c[kMergeChunk];
    load_chunk(c, 0);

    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < kMaxSplits / 256; ++u) mx = fmaxf(mx, mlv[u].x);
    const float M = block_max256(mx, red);  // finite: every split has a token
    float ls = 0.f;
#pragma unroll
    for (int u = 0; u < kMaxSplits / 256; ++u) {
        const int sidx = tid + 256 * u;
        if (sidx < a.NS) {
            const float e = exp2f(mlv[u].x - M);
            wsplit[sidx] = e;
            ls += e * mlv[u].y;
        }
    }
    const float inv_l = 1.0f / block_sum256(ls, red);  // block_sum256 synchronises wsplit

    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s0 = 0;;) {
#pragma unroll
        for (int u = 0; u < kMergeChunk; ++u) {
            const int sidx = s0 + 8 * u + g;
            const float ws = sidx < a.NS ? wsplit[sidx] : 0.f;
            acc.x = fmaf(ws, c[u].x, acc.x);
            acc.y = fmaf(ws, c[u].y, acc.y);
            acc.z = fmaf(ws, c[u].z, acc.z);
            acc.w = fmaf(ws, c[u].w, acc.w);
        }
        s0 += 8 * kMergeChunk;
        if (s0 >= a.NS) break;
        load_chunk(c, s0);
    }
    red8[g][c4] = acc;
    __syncthreads();
    if (tid < kMQCols / 4) {
        float4 t = red8[0][tid];
#pragma unroll
        for (int j = 1; j < 8; ++j) {
            const float4 o = red8[j][tid];
            t.x += o.x, t.y += o.y, t.z += o.z, t.w += o.w;
        }
        *reinterpret_cast<float4 *>(ctx + 4 * tid) = make_float4(t.x * inv_l, t.y * inv_l, t.z * inv_l, t.w * inv_l);
    }
    __syncthreads();

    const float4 x0 = *reinterpret_cast<const float4 *>(ctx + sub * 8);
    const float4 x1 = *reinterpret_cast<const float4 *>(ctx + sub * 8 + 4);
    const float x8[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    float *orow = a.opart + (static_cast<int64_t>(q) * a.H + h) * a.V;
    for (int vb = 0; vb < a.V; vb += 16 * kUvBatch) {
        if (vb > 0) {
#pragma unroll
            for (int i = 0; i < kUvBatch; ++i) w[i] = w_row(vb + 16 * i + vrow);
        }
#pragma unroll
        for (int i = 0; i < kUvBatch; ++i) {
            const uint32_t wd[4] = {w[i].x, w[i].y, w[i].z, w[i].w};
            float o = 0.f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                o = fmaf(__uint_as_float(wd[k] << 16), x8[2 * k], o);
                o = fmaf(__uint_as_float(wd[k] & 0xffff0000u), x8[2 * k + 1], o);
            }
            o = row16_sum(o);
            const int v = vb + 16 * i + vrow;
            if (sub == 0 && v < a.V) orow[v] = o;
        }
    }
}

struct OutArgs {
    const float *opart;  // [4, H, V]
    void *out;           // [H, V] rows of ld_out elements
    int64_t ld_out;
    int H, V;
    int out_bf16;
    const float *gate;   // [H, V] logits or null: o *= sigmoid(gate) (the MLA output gate)
};

// o[h][v] = the four column-quarter products added in quarter order (then the output gate)
__global__ __launch_bounds__(256) void mla_out_kernel(OutArgs a) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int n = a.H * a.V;
    if (i >= n) return;
    float o = a.opart[i];
#pragma unroll
    for (int q = 1; q < kMergeQ; ++q) o += a.opart[static_cast<int64_t>(q) * n + i];
    if (a.gate) o /= 1.0f + expf(-a.gate[i]);
    const int h = i / a.V, v = i % a.V;
    const int64_t oi = static_cast<int64_t>(h) * a.ld_out + v;
    if (a.out_bf16)
        static_cast<uint16_t *>(a.out)[oi] = f32_to_bf16(o);
    else
        static_cast<float *>(a.out)[oi] = o;
}

// ------------------------------------------------------------------ host side
#ifndef K3_MLA_D
#define K3_MLA_D 2
#endif
constexpr int kD = K3_MLA_D;  // staged rounds in flight

// One attention block per CU: about 256 blocks of (head group, split); a split is a
// multiple of one round of tiles.
void mla_splits(int64_t H, int64_t T, int *Ts, int *NS) {
    const int64_t hgn = cdiv(H, kHG);
    const int64_t want = std::max<int64_t>(1, 256 / hgn);
    int64_t ts = cdiv(T, want);
    ts = cdiv(ts, kStepT * kRoundTiles) * kStepT * kRoundTiles;
    *Ts = static_cast<int>(ts);
    *NS = static_cast<int>(cdiv(T, ts));
}

constexpr int kMaxV = 1024;  // largest v_head_dim the merge takes

struct MlaWs {
    size_t qa_hi, qa_lo, ml, part, opart, total;
};

MlaWs mla_ws_layout(int64_t H, int64_t T) {
    int Ts, NS;
    mla_splits(H, std::max<int64_t>(T, 1), &Ts, &NS);
    MlaWs L{};
    auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
    size_t o = 0;
    L.qa_hi = o, o += up(static_cast<size_t>(H) * kQaLd * 2);
    L.qa_lo = o, o += up(static_cast<size_t>(H) * kQaLd * 2);
    L.ml = o, o += up(static_cast<size_t>(NS) * H * 8);
    L.part = o, o += up(static_cast<size_t>(NS) * H * kR * 4);
    L.opart = o, o += up(static_cast<size_t>(kMergeQ) * H * kMaxV * 4);
    L.total = o;
    return L;
}

}  // namespace
}  // namespace k3

using namespace k3;

extern "C" int64_t k3_mla_workspace_size(int64_t H, int64_t T) {
    if (H <= 0 || T < 0) return 0;
    return static_cast<int64_t>(mla_ws_layout(H, T).total);
}

extern "C" int k3_mla_decode_absorbed(const void *q_nope, const void *q_rot, int64_t ld_q, int64_t ld_q_rot,
                                      int q_dtype, const void *w_uk, const void *w_uv, const void *lat, int64_t ld_lat,
                                      const void *rot, int64_t ld_rot, int64_t T, int64_t H, int64_t kv_lora_rank,
                                      int64_t rope_dim, int64_t nope_dim, int64_t v_dim, float scale, void *out,
                                      int out_dtype, int64_t ld_out, void *workspace, int64_t workspace_bytes,
                                      void *stream) {
    return k3::mla_decode_core(q_nope, q_rot, ld_q, ld_q_rot, q_dtype, w_uk, w_uv, lat, ld_lat, rot, ld_rot, T, H,
                               kv_lora_rank, rope_dim, nope_dim, v_dim, scale, out, out_dtype, ld_out, nullptr,
                               workspace, workspace_bytes, stream, K3_BF16);
}

extern "C" int k3_mla_decode_absorbed_f32(const void *q_nope, const void *q_rot, int64_t ld_q, int64_t ld_q_rot,
                                          int q_dtype, const void *w_uk, const void *w_uv, const void *lat,
                                          int64_t ld_lat, const void *rot, int64_t ld_rot, int64_t T, int64_t H,
                                          int64_t kv_lora_rank, int64_t rope_dim, int64_t nope_dim, int64_t v_dim,
                                          float scale, void *out, int out_dtype, int64_t ld_out, void *workspace,
                                          int64_t workspace_bytes, void *stream) {
    return k3::mla_decode_core(q_nope, q_rot, ld_q, ld_q_rot, q_dtype, w_uk, w_uv, lat, ld_lat, rot, ld_rot, T, H,
                               kv_lora_rank, rope_dim, nope_dim, v_dim, scale, out, out_dtype, ld_out, nullptr,
                               workspace, workspace_bytes, stream, K3_F32);
}

int k3::mla_decode_core(const void *q_nope, const void *q_rot, int64_t ld_q, int64_t ld_q_rot, int q_dtype,
                        const void *w_uk, const void *w_uv, const void *lat, int64_t ld_lat, const void *rot,
                        int64_t ld_rot, int64_t T, int64_t H, int64_t kv_lora_rank, int64_t rope_dim,
                        int64_t nope_dim, int64_t v_dim, float scale, void *out, int out_dtype, int64_t ld_out,
                        const float *gate, void *workspace, int64_t workspace_bytes, void *stream, int cache_dtype) {
    if (!q_nope || !q_rot || !w_uk || !w_uv || !lat || !rot || !out || !workspace)
        return set_error(K3_ERR_NULL, "mla decode: null pointer");
    if (q_dtype != K3_F32 && q_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "mla decode: q_dtype %d", q_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "mla decode: out_dtype %d", out_dtype);
    if (cache_dtype != K3_F32 && cache_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "mla decode: cache dtype %d", cache_dtype);
    const bool f32c = cache_dtype == K3_F32;
    const int64_t esz = f32c ? 4 : 2, align_el = 16 / esz;  // cache element bytes; elements per 16 bytes
    if (kv_lora_rank != kR || rope_dim != kRope)
        return set_error(K3_ERR_SHAPE, "mla decode: kv_lora_rank=%lld rope=%lld; the kernels take 512 and 64",
                         (long long)kv_lora_rank, (long long)rope_dim);
    if (H <= 0 || H > 4096) return set_error(K3_ERR_SHAPE, "mla decode: H=%lld must be in 1..4096", (long long)H);
    if (nope_dim <= 0 || nope_dim > 256 || v_dim <= 0 || v_dim > kMaxV)
        return set_error(K3_ERR_SHAPE, "mla decode: nope=%lld must be in 1..256 and v=%lld in 1..1024",
                         (long long)nope_dim, (long long)v_dim);
    if (T <= 0) return set_error(K3_ERR_SHAPE, "mla decode: empty cache (T=%lld)", (long long)T);
    if (ld_q < nope_dim || ld_q_rot < rope_dim || ld_lat < kR || ld_rot < kRope || ld_out < v_dim ||
        ld_lat % align_el || ld_rot % align_el)
        return set_error(K3_ERR_SHAPE, "mla decode: row strides too small, or cache rows not 16-byte multiples");
    if (!aligned16(lat) || !aligned16(rot) || !aligned16(w_uk) || !aligned16(w_uv) || !aligned16(workspace))
        return set_error(K3_ERR_ALIGN, "mla decode: cache, weights and workspace must be 16-byte aligned");
    const int64_t lat_bytes = ((T - 1) * ld_lat + kR) * esz, rot_bytes = ((T - 1) * ld_rot + kRope) * esz;
    if (lat_bytes >= (1ll << 31) || rot_bytes >= (1ll << 31))
        return set_error(K3_ERR_SHAPE, "mla decode: cache views above 2 GiB are not supported");
    const MlaWs L = mla_ws_layout(H, T);
    if (workspace_bytes < static_cast<int64_t>(L.total))
        return set_error(K3_ERR_WORKSPACE, "mla decode: workspace %lld < %zu bytes", (long long)workspace_bytes,
                         L.total);
    int Ts, NS;
    mla_splits(H, T, &Ts, &NS);
    if (NS > kMaxSplits) return set_error(K3_ERR_SHAPE, "mla decode: T=%lld needs too many splits", (long long)T);
    auto st = static_cast<hipStream_t>(stream);
    char *ws = static_cast<char *>(workspace);
    uint16_t *qa_hi = reinterpret_cast<uint16_t *>(ws + L.qa_hi);
    uint16_t *qa_lo = reinterpret_cast<uint16_t *>(ws + L.qa_lo);
    float *part = reinterpret_cast<float *>(ws + L.part);
    float2 *ml = reinterpret_cast<float2 *>(ws + L.ml);

    QaArgs qa{q_nope, q_rot, ld_q, ld_q_rot, static_cast<const uint16_t *>(w_uk), qa_hi, qa_lo, static_cast<int>(H),
              static_cast<int>(nope_dim)};
    if (q_dtype == K3_BF16)
        mla_qa_kernel<uint16_t><<<dim3(static_cast<unsigned>(H * 4)), 256, 0, st>>>(qa);
    else
        mla_qa_kernel<float><<<dim3(static_cast<unsigned>(H * 4)), 256, 0, st>>>(qa);
    int rc = check_hip(hipGetLastError(), "mla decode: qa launch");
    if (rc) return rc;

    AttnArgs aa{};
    aa.qa_hi = qa_hi;
    aa.qa_lo = qa_lo;
    aa.lat = lat;
    aa.rot = rot;
    aa.lat_bytes = static_cast<uint32_t>(lat_bytes);
    aa.rot_bytes = static_cast<uint32_t>(rot_bytes);
    aa.lat_row_bytes = static_cast<uint32_t>(ld_lat * esz);
    aa.rot_row_bytes = static_cast<uint32_t>(ld_rot * esz);
    aa.part = part;
    aa.ml = ml;
    aa.H = static_cast<int>(H);
    aa.T = static_cast<int>(T);
    aa.Ts = Ts;
    aa.NS = NS;
    aa.scale_log2 = scale * 1.4426950408889634f;
    const int blocks = NS * static_cast<int>(cdiv(H, kHG));
    aa.swizzle = blocks % 8 == 0;
    constexpr auto attn_bf16 = &mla_attn_kernel<kD, false>;
    constexpr auto attn_f32 = &mla_attn_kernel<kD, true>;
    constexpr size_t lds = kAttnLds;
    // may exceed the 64 KB default; set once per process for each form
    static const hipError_t lds_rc =
        hipFuncSetAttribute(reinterpret_cast<const void *>(attn_bf16), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds));
    static const hipError_t lds_rc32 =
        hipFuncSetAttribute(reinterpret_cast<const void *>(attn_f32), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds));
    rc = check_hip(f32c ? lds_rc32 : lds_rc, "mla decode: attention LDS size");
    if (rc) return rc;
    if (f32c)
        attn_f32<<<dim3(static_cast<unsigned>(blocks)), 512, lds, st>>>(aa);
    else
        attn_bf16<<<dim3(static_cast<unsigned>(blocks)), 512, lds, st>>>(aa);
    rc = check_hip(hipGetLastError(), "mla decode: attention launch");
    if (rc) return rc;

    float *opart = reinterpret_cast<float *>(ws + L.opart);
    MergeArgs ma{part, ml, static_cast<const uint16_t *>(w_uv), opart, static_cast<int>(H), NS,
                 static_cast<int>(v_dim)};
    mla_merge_kernel<<<dim3(static_cast<unsigned>(H * kMergeQ)), 256, 0, st>>>(ma);
    rc = check_hip(hipGetLastError(), "mla decode: merge and W_UV launch");
    if (rc) return rc;
    OutArgs oa{opart, out, ld_out, static_cast<int>(H), static_cast<int>(v_dim), out_dtype == K3_BF16, gate};
    mla_out_kernel<<<dim3(static_cast<unsigned>(cdiv(H * v_dim, 256))), 256, 0, st>>>(oa);
    return check_hip(hipGetLastError(), "mla decode: output launch");
}
