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
//   A   split-T flash decoding.  A block owns 32 heads and a contiguous token range; it
//       walks the range in 32-token tiles: the tile goes HBM -> registers (prefetched one
//       tile ahead) -> LDS; scores S[32 heads x 32 tokens] come from bf16 MFMAs
//       (v_mfma_f32_16x16x32_bf16) of the hi and the lo half of qa against the tile; an
//       online softmax (base 2, running max and sum per head) turns them into P, split
//       again into a bf16 hi/lo pair; ctx[32 x 512] += P_hi @ tile + P_lo @ tile on MFMA.
//       The block writes its unnormalised (ctx, max, sum) record per head.
//   M   per (head, quarter of the latent columns): log-sum-exp merge of the split records
//       in a fixed order into the normalised ctx.
//   U   o = W_UV[h] @ ctx[h] in fp32, 32 output rows per block.
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
constexpr int kLdsRow = kK + 8;  // padded LDS row (1168 B): conflict-free 16-byte row reads
constexpr int kTile = 32;        // tokens per tile
constexpr int kHG = 16;          // heads per attention block (one MFMA row tile)
constexpr int kPRow = kTile + 8; // padded P row (bf16)
constexpr int kSRow = kTile + 1; // padded score row (fp32)
constexpr int kPartLd = 516;     // floats per (split, head) record: ctx[512], max, sum, pad
constexpr int kMaxSplits = 1024;
constexpr int kChunksPerRow = kK / 8;  // 16-byte chunks per token row (64 lat + 8 rot)
constexpr int kPre = kTile * kChunksPerRow / 256;  // chunks per thread per tile (9)
constexpr int kKSteps = kK / 32;                   // 18 MFMA k-steps over the score contraction

// tile, P hi/lo, two partial-score planes, running max / sum / rescale
constexpr size_t kAttnLds = kTile * kLdsRow * 2 + 2 * kHG * kPRow * 2 + 2 * kHG * kSRow * 4 + 3 * kHG * 4;

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
    const void *q_nope, *q_rot;  // [H, ld_q] rows (bf16 or fp32)
    int64_t ld_q;
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
        const float v = load_q(static_cast<const QT *>(a.q_rot) + static_cast<int64_t>(h) * a.ld_q + j);
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
    int64_t ld_lat, ld_rot;         // elements between tokens
    float *part;                    // [NS, H, kPartLd]
    int H, T, Ts, NS;
    float scale_log2;               // softmax scale * log2(e)
    int swizzle;                    // XCD-aware block -> work mapping
};

// Block: 16 heads x one split (tiles s, s + NS, ...); 4 waves; ~44 KB of LDS and <= 128
// VGPRs + AGPRs per lane, so two blocks share a CU and hide each other's barriers.
//   scores  wave (nt, kh): tokens 16 nt .. +16 of the tile, k-steps 9 kh .. +9; its qa
//           operands (hi and lo) live in registers for the whole kernel
//   softmax 16 threads per head, 2 tokens each, over the two k-half planes
//   ctx     wave w: latent columns 128 w .. +128 (8 MFMA column tiles); the transposed tile
//           operand comes from ds_read_b64_tr_b16 (two per MFMA)
__global__ __launch_bounds__(256, 2) void mla_attn_kernel(AttnArgs a) {
    extern __shared__ uint4 smem[];
    uint16_t *lat_s = reinterpret_cast<uint16_t *>(smem);                 // [32][kLdsRow]
    uint16_t *p_s = lat_s + kTile * kLdsRow;                                // [2][16][kPRow]
    float *s_s = reinterpret_cast<float *>(p_s + 2 * kHG * kPRow);          // [2][16][kSRow]
    float *m_run = s_s + 2 * kHG * kSRow;
    float *l_run = m_run + kHG;
    float *alpha = l_run + kHG;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // blocks b, b+8, b+16, ... share an XCD (and its L2): give them consecutive work items,
    // so the head groups of one split read the same tiles through one L2
    const int b = blockIdx.x;
    const int w = a.swizzle ? (b & 7) * (static_cast<int>(gridDim.x) >> 3) + (b >> 3) : b;
    const int HGn = (a.H + kHG - 1) / kHG;
    const int hg = w % HGn, split = w / HGn;
    const int h0 = hg * kHG;
    // Split s owns the 32-token tiles s, s + NS, s + 2 NS, ...: blocks that run together
    // read neighbouring tiles.
    const int n_all = (a.T + kTile - 1) / kTile;
    const int ntiles = (n_all - split + a.NS - 1) / a.NS;  // >= 1: NS <= n_all
    auto tile_base = [&](int it) { return (split + it * a.NS) * kTile; };

    const auto rl = make_rsrc(a.lat, a.lat_bytes);
    const auto rr = make_rsrc(a.rot, a.rot_bytes);
    // tile = 32 rows of 64 latent chunks + 32 rows of 8 rope chunks (16 B each): 8 latent
    // loads and 1 rope load per thread, each a uniform instruction over the wave
    auto load_tile = [&](uint4(&buf)[kPre], int tb) {
#pragma unroll
        for (int i = 0; i < kPre - 1; ++i) {
            const int c = tid + 256 * i;
            const int t = tb + (c >> 6);
            buf[i] = buf_load16(rl, t < a.T ? static_cast<uint32_t>(t * a.ld_lat * 2 + (c & 63) * 16) : kOobOffset);
        }
        const int t = tb + (tid >> 3);
        buf[kPre - 1] = buf_load16(rr, t < a.T ? static_cast<uint32_t>(t * a.ld_rot * 2 + (tid & 7) * 16) : kOobOffset);
    };
    uint4 pre0[kPre];
    load_tile(pre0, tile_base(0));

    // this wave's qa operands: head h0 + (lane % 16), k-steps 9 kh .. 9 kh + 8 (L2-resident)
    const int r16 = lane & 15, q4 = lane >> 4;
    const int nt = wave & 1, kh = wave >> 1;
    // heads past H (last group) load zeros (out-of-range buffer offsets) and score 0; no
    // select on the loaded values, so nothing waits for these loads before the first tile
    bf16x8 qhi[kKSteps / 2], qlo[kKSteps / 2];
    {
        const uint32_t qbytes = static_cast<uint32_t>(a.H) * kQaLd * 2;
        const auto rqh = make_rsrc(a.qa_hi, qbytes), rql = make_rsrc(a.qa_lo, qbytes);
        const uint32_t qoff = h0 + r16 < a.H ? static_cast<uint32_t>(((h0 + r16) * kQaLd + kh * (kK / 2) + q4 * 8) * 2)
                                             : kOobOffset;
#pragma unroll
        for (int k = 0; k < kKSteps / 2; ++k) {
            qhi[k] = __builtin_bit_cast(bf16x8, buf_load16(rqh, qoff + k * 64u));
            qlo[k] = __builtin_bit_cast(bf16x8, buf_load16(rql, qoff + k * 64u));
        }
    }
    if (tid < kHG) {
        m_run[tid] = -INFINITY;
        l_run[tid] = 0.f;
    }

    f32x4_t cacc[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) cacc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto tile_step = [&](int it, uint4(&buf)[kPre]) {
        const int tb = tile_base(it);
        __syncthreads();  // previous tile's LDS reads are done
#pragma unroll
        for (int i = 0; i < kPre - 1; ++i) {
            const int c = tid + 256 * i;
            *reinterpret_cast<uint4 *>(lat_s + (c >> 6) * kLdsRow + (c & 63) * 8) = buf[i];
        }
        *reinterpret_cast<uint4 *>(lat_s + (tid >> 3) * kLdsRow + kR + (tid & 7) * 8) = buf[kPre - 1];
        __syncthreads();
        if (it + 1 < ntiles) load_tile(buf, tile_base(it + 1));

        // ---- partial scores over this wave's k half (hi and lo chains)
        {
            const uint16_t *bp = lat_s + (nt * 16 + r16) * kLdsRow + kh * (kK / 2) + q4 * 8;
            f32x4_t sh = {0.f, 0.f, 0.f, 0.f}, sl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < kKSteps / 2; ++k) {
                const bf16x8 bv = *reinterpret_cast<const bf16x8 *>(bp + k * 32);
                sh = mfma_bf16(qhi[k], bv, sh);
                sl = mfma_bf16(qlo[k], bv, sl);
            }
            const f32x4_t st = sh + sl;
            float *sp = s_s + kh * kHG * kSRow;
#pragma unroll
            for (int i = 0; i < 4; ++i) sp[(q4 * 4 + i) * kSRow + nt * 16 + r16] = st[i];
        }
        __syncthreads();

        // ---- online softmax: 16 threads per head, 2 tokens each
        {
            const int hh = tid >> 4, q = tid & 15;
            float sv[2];
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int tok = q * 2 + j;
                const float v = (s_s[hh * kSRow + tok] + s_s[(kHG + hh) * kSRow + tok]) * a.scale_log2;
                sv[j] = tb + tok < a.T ? v : -INFINITY;
                mx = fmaxf(mx, sv[j]);
            }
            mx = row16_max(mx);
            const float mold = m_run[hh];
            const float mnew = fmaxf(mold, mx);  // finite: every tile holds a valid token
            float ps = 0.f;
            uint16_t *ph = p_s + hh * kPRow + q * 2;
            uint16_t *pl = ph + kHG * kPRow;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float p = exp2f(sv[j] - mnew);
                ps += p;
                split_bf16(p, ph[j], pl[j]);
            }
            ps = row16_sum(ps);
            if (q == 0) {
                const float al = exp2f(mold - mnew);
                alpha[hh] = al;
                l_run[hh] = l_run[hh] * al + ps;
                m_run[hh] = mnew;
            }
        }
        __syncthreads();

        // ---- ctx[16 x 512] += P @ tile: wave owns latent columns [128 wave, +128)
        {
            const bf16x8 ph = *reinterpret_cast<const bf16x8 *>(p_s + r16 * kPRow + q4 * 8);
            const bf16x8 pl = *reinterpret_cast<const bf16x8 *>(p_s + (kHG + r16) * kPRow + q4 * 8);
            float al[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) al[i] = alpha[q4 * 4 + i];
            if (!__all(al[0] == 1.f && al[1] == 1.f && al[2] == 1.f && al[3] == 1.f)) {
#pragma unroll
                for (int n = 0; n < 8; ++n)
#pragma unroll
                    for (int i = 0; i < 4; ++i) cacc[n][i] *= al[i];
            }
            // transposed operand: source lane s' of group g points at token 8g + s'/4,
            // columns c0 + 4 (s' % 4) .. +3; a second read 4 tokens further down
            typedef short s4_t __attribute__((ext_vector_type(4)));
            const uint16_t *tsrc = lat_s + (q4 * 8 + (r16 >> 2)) * kLdsRow + wave * 128 + (r16 & 3) * 4;
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                typedef __attribute__((address_space(3))) s4_t *lds_s4;
                const s4_t lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(tsrc + n * 16));
                const s4_t hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(tsrc + n * 16 + 4 * kLdsRow));
                const bf16x8 bb = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
                cacc[n] = mfma_bf16(ph, bb, cacc[n]);
                cacc[n] = mfma_bf16(pl, bb, cacc[n]);
            }
        }
    };
    for (int it = 0; it < ntiles; ++it) tile_step(it, pre0);

    // ---- split record: unnormalised ctx, running max and sum
    float *part = a.part + (static_cast<int64_t>(split) * a.H + h0) * kPartLd;
#pragma unroll
    for (int n = 0; n < 8; ++n)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (h0 + q4 * 4 + i < a.H) part[(q4 * 4 + i) * kPartLd + wave * 128 + n * 16 + r16] = cacc[n][i];
    if (tid < kHG && h0 + tid < a.H) {
        part[tid * kPartLd + kR] = m_run[tid];
        part[tid * kPartLd + kR + 1] = l_run[tid];
    }
}

// ------------------------------------------------------------------ M: merge, then W_UV
struct MergeArgs {
    const float *part;
    float *ctx;            // [H, 512] merged, normalised context
    const uint16_t *w_uv;  // [H, V, 512] bf16
    void *out;             // [H, V] rows of ld_out elements
    int64_t ld_out;
    int H, NS, V;
    int out_bf16;
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

// grid: H * 4; block (h, quarter): ctx[h][128 quarter .. +128) = sum_s w_s ctx_s / L with
// w_s = 2^(m_s - M).  Fixed order: 8 groups of splits (s = g mod 8), then the groups in order.
// Every load of a thread is issued before the first is used: the records come from the
// last-level cache, so the cost is round trips, not bytes.
__global__ __launch_bounds__(256) void mla_merge_kernel(MergeArgs a) {
    __shared__ float wsplit[kMaxSplits];
    __shared__ float csum[8][129];
    __shared__ float red[4];
    const int h = blockIdx.x >> 2, quarter = blockIdx.x & 3;
    const int tid = threadIdx.x;
    const float *rec = a.part + static_cast<int64_t>(h) * kPartLd;
    const int64_t sstride = static_cast<int64_t>(a.H) * kPartLd;

    // column loads first (16 splits per thread covers NS <= 128 in one batch)
    const int c4 = tid & 31, grp = tid >> 5;
    const float *col = rec + quarter * 128 + 4 * c4;
    constexpr int kPer = 16;
    float4 v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int s = grp + 8 * u;
        v[u] = s < a.NS ? *reinterpret_cast<const float4 *>(col + s * sstride) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float mv[kMaxSplits / 256], lv[kMaxSplits / 256];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kMaxSplits / 256; ++j) {
        const int s = tid + 256 * j;
        mv[j] = s < a.NS ? rec[s * sstride + kR] : -INFINITY;
        lv[j] = s < a.NS ? rec[s * sstride + kR + 1] : 0.f;
        mx = fmaxf(mx, mv[j]);
    }
    const float M = block_max256(mx, red);
    float ls = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxSplits / 256; ++j) {
        const int s = tid + 256 * j;
        if (s < a.NS) {
            const float e = exp2f(mv[j] - M);
            wsplit[s] = e;
            ls += e * lv[j];
        }
    }
    const float inv_l = 1.0f / block_sum256(ls, red);  // block_sum256 synchronises wsplit

    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int s = grp + 8 * u;
        const float ws = s < a.NS ? wsplit[s] : 0.f;
        acc.x = fmaf(ws, v[u].x, acc.x);
        acc.y = fmaf(ws, v[u].y, acc.y);
        acc.z = fmaf(ws, v[u].z, acc.z);
        acc.w = fmaf(ws, v[u].w, acc.w);
    }
    for (int s0 = grp + 8 * kPer; s0 < a.NS; s0 += 8 * kPer) {  // NS > 128
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int s = s0 + 8 * u;
            v[u] = s < a.NS ? *reinterpret_cast<const float4 *>(col + s * sstride) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int s = s0 + 8 * u;
            const float ws = s < a.NS ? wsplit[s] : 0.f;
            acc.x = fmaf(ws, v[u].x, acc.x);
            acc.y = fmaf(ws, v[u].y, acc.y);
            acc.z = fmaf(ws, v[u].z, acc.z);
            acc.w = fmaf(ws, v[u].w, acc.w);
        }
    }
    csum[grp][4 * c4] = acc.x;
    csum[grp][4 * c4 + 1] = acc.y;
    csum[grp][4 * c4 + 2] = acc.z;
    csum[grp][4 * c4 + 3] = acc.w;
    __syncthreads();
    if (tid < 128) {
        float r = 0.f;
        for (int g = 0; g < 8; ++g) r += csum[g][tid];
        a.ctx[h * kR + quarter * 128 + tid] = r * inv_l;
    }
}

// grid: cdiv(H * V, 32); block: 32 output rows (8 per wave) of o[h][v] = W_UV[h][v] . ctx[h];
// lane l covers columns 8l .. 8l+7, all 8 rows' weights in flight at once
__global__ __launch_bounds__(256) void mla_uv_kernel(MergeArgs a) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t rows = static_cast<int64_t>(a.H) * a.V;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 32 + wave * 8;
    uint4 w[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int64_t r = r0 + u;
        w[u] = r < rows ? *reinterpret_cast<const uint4 *>(a.w_uv + r * kR + lane * 8) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int64_t r = r0 + u;
        const int h = static_cast<int>(min(r, rows - 1) / a.V);
        const float4 c0 = *reinterpret_cast<const float4 *>(a.ctx + h * kR + lane * 8);
        const float4 c1 = *reinterpret_cast<const float4 *>(a.ctx + h * kR + lane * 8 + 4);
        const float c8[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        const uint32_t wd[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
        float acc = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc = fmaf(__uint_as_float(wd[q] << 16), c8[2 * q], acc);
            acc = fmaf(__uint_as_float(wd[q] & 0xffff0000u), c8[2 * q + 1], acc);
        }
        acc = wave_sum_to_lane63(acc);
        if (lane == 63 && r < rows) {
            const int64_t oi = static_cast<int64_t>(h) * a.ld_out + (r - static_cast<int64_t>(h) * a.V);
            if (a.out_bf16)
                static_cast<uint16_t *>(a.out)[oi] = f32_to_bf16(acc);
            else
                static_cast<float *>(a.out)[oi] = acc;
        }
    }
}

// ------------------------------------------------------------------ host side
// Tokens per split: at least 128 (the qa tile staged per block is amortised over >= 4
// tiles), otherwise enough that one split per 128 tokens-of-work keeps ~256 blocks busy.
void mla_splits(int64_t T, int *Ts, int *NS) {
    int64_t ts = std::max<int64_t>(128, cdiv(T, 128));
    ts = cdiv(ts, kTile) * kTile;
    *Ts = static_cast<int>(ts);
    *NS = static_cast<int>(cdiv(T, ts));
}

struct MlaWs {
    size_t qa_hi, qa_lo, ctx, part, total;
};

MlaWs mla_ws_layout(int64_t H, int64_t T) {
    int Ts, NS;
    mla_splits(std::max<int64_t>(T, 1), &Ts, &NS);
    MlaWs L{};
    auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
    size_t o = 0;
    L.qa_hi = o, o += up(static_cast<size_t>(H) * kQaLd * 2);
    L.qa_lo = o, o += up(static_cast<size_t>(H) * kQaLd * 2);
    L.ctx = o, o += up(static_cast<size_t>(H) * kR * 4);
    L.part = o, o += up(static_cast<size_t>(NS) * H * kPartLd * 4);
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

extern "C" int k3_mla_decode_absorbed(const void *q_nope, const void *q_rot, int64_t ld_q, int q_dtype,
                                      const void *w_uk, const void *w_uv, const void *lat, int64_t ld_lat,
                                      const void *rot, int64_t ld_rot, int64_t T, int64_t H, int64_t kv_lora_rank,
                                      int64_t rope_dim, int64_t nope_dim, int64_t v_dim, float scale, void *out,
                                      int out_dtype, int64_t ld_out, void *workspace, int64_t workspace_bytes,
                                      void *stream) {
    if (!q_nope || !q_rot || !w_uk || !w_uv || !lat || !rot || !out || !workspace)
        return set_error(K3_ERR_NULL, "mla decode: null pointer");
    if (q_dtype != K3_F32 && q_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "mla decode: q_dtype %d", q_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "mla decode: out_dtype %d", out_dtype);
    if (kv_lora_rank != kR || rope_dim != kRope)
        return set_error(K3_ERR_SHAPE, "mla decode: kv_lora_rank=%lld rope=%lld; the kernels take 512 and 64",
                         (long long)kv_lora_rank, (long long)rope_dim);
    if (H <= 0 || H > 4096) return set_error(K3_ERR_SHAPE, "mla decode: H=%lld must be in 1..4096", (long long)H);
    if (nope_dim <= 0 || nope_dim > 256 || v_dim <= 0 || v_dim > 1024)
        return set_error(K3_ERR_SHAPE, "mla decode: nope=%lld must be in 1..256 and v=%lld in 1..1024",
                         (long long)nope_dim, (long long)v_dim);
    if (T <= 0) return set_error(K3_ERR_SHAPE, "mla decode: empty cache (T=%lld)", (long long)T);
    if (ld_q < nope_dim || ld_lat < kR || ld_rot < kRope || ld_out < v_dim || ld_lat % 8 || ld_rot % 8)
        return set_error(K3_ERR_SHAPE, "mla decode: row strides too small, or cache strides not multiples of 8");
    if (!aligned16(lat) || !aligned16(rot) || !aligned16(w_uk) || !aligned16(w_uv) || !aligned16(workspace))
        return set_error(K3_ERR_ALIGN, "mla decode: cache, weights and workspace must be 16-byte aligned");
    const int64_t lat_bytes = ((T - 1) * ld_lat + kR) * 2, rot_bytes = ((T - 1) * ld_rot + kRope) * 2;
    if (lat_bytes >= (1ll << 31) || rot_bytes >= (1ll << 31))
        return set_error(K3_ERR_SHAPE, "mla decode: cache views above 2 GiB are not supported");
    const MlaWs L = mla_ws_layout(H, T);
    if (workspace_bytes < static_cast<int64_t>(L.total))
        return set_error(K3_ERR_WORKSPACE, "mla decode: workspace %lld < %zu bytes", (long long)workspace_bytes,
                         L.total);
    int Ts, NS;
    mla_splits(T, &Ts, &NS);
    if (NS > kMaxSplits) return set_error(K3_ERR_SHAPE, "mla decode: T=%lld needs too many splits", (long long)T);
    auto st = static_cast<hipStream_t>(stream);
    char *ws = static_cast<char *>(workspace);
    uint16_t *qa_hi = reinterpret_cast<uint16_t *>(ws + L.qa_hi);
    uint16_t *qa_lo = reinterpret_cast<uint16_t *>(ws + L.qa_lo);
    float *part = reinterpret_cast<float *>(ws + L.part);

    QaArgs qa{q_nope, q_rot, ld_q, static_cast<const uint16_t *>(w_uk), qa_hi, qa_lo, static_cast<int>(H),
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
    aa.ld_lat = ld_lat;
    aa.ld_rot = ld_rot;
    aa.part = part;
    aa.H = static_cast<int>(H);
    aa.T = static_cast<int>(T);
    aa.Ts = Ts;
    aa.NS = NS;
    aa.scale_log2 = scale * 1.4426950408889634f;
    const int blocks = NS * static_cast<int>(cdiv(H, kHG));
    aa.swizzle = blocks % 8 == 0;
    static_assert(kAttnLds <= 64 * 1024, "attention LDS: two blocks per CU");
    mla_attn_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, kAttnLds, st>>>(aa);
    rc = check_hip(hipGetLastError(), "mla decode: attention launch");
    if (rc) return rc;

    MergeArgs ma{part, reinterpret_cast<float *>(ws + L.ctx), static_cast<const uint16_t *>(w_uv), out, ld_out,
                 static_cast<int>(H), NS, static_cast<int>(v_dim), out_dtype == K3_BF16};
    mla_merge_kernel<<<dim3(static_cast<unsigned>(H * 4)), 256, 0, st>>>(ma);
    rc = check_hip(hipGetLastError(), "mla decode: merge launch");
    if (rc) return rc;
    mla_uv_kernel<<<dim3(static_cast<unsigned>(cdiv(H * v_dim, 32))), 256, 0, st>>>(ma);
    return check_hip(hipGetLastError(), "mla decode: W_UV launch");
}
