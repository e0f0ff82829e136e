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
// Here the cache stays bf16 and is read once; three stream-ordered launches:
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
//   M   per (head, 32 output rows): log-sum-exp merge of the split records in a fixed
//       order, then o = W_UV[h] @ ctx in fp32.
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
constexpr int kHG = 32;          // heads per attention block
constexpr int kPRow = kTile + 8; // padded P row (bf16)
constexpr int kSRow = kTile + 1; // padded score row (fp32)
constexpr int kPartLd = 516;     // floats per (split, head) record: ctx[512], max, sum, pad
constexpr int kMaxSplits = 1024;
constexpr int kChunksPerRow = kK / 8;  // 16-byte chunks per token row (64 lat + 8 rot)
constexpr int kPre = kTile * kChunksPerRow / 256;  // chunks per thread per tile (9)

constexpr size_t kAttnLds = (2 * kHG + kTile) * kLdsRow * 2 + 2 * kHG * kPRow * 2 +
                            kHG * kSRow * 4 + 3 * kHG * 4;

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma_bf16(bf16x8 a, bf16x8 b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
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
    for (int n = ng; n < a.nope; n += 16) {
        const uint4 w = *reinterpret_cast<const uint4 *>(wrow + static_cast<int64_t>(n) * kR);
        const float qv = qn[n];
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
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

__global__ __launch_bounds__(256) void mla_attn_kernel(AttnArgs a) {
    extern __shared__ uint4 smem[];
    uint16_t *qa_s = reinterpret_cast<uint16_t *>(smem);          // [2][32][kLdsRow]
    uint16_t *lat_s = qa_s + 2 * kHG * kLdsRow;                     // [32][kLdsRow]
    uint16_t *p_s = lat_s + kTile * kLdsRow;                        // [2][32][kPRow]
    float *s_s = reinterpret_cast<float *>(p_s + 2 * kHG * kPRow);  // [32][kSRow]
    float *m_run = s_s + kHG * kSRow;
    float *l_run = m_run + kHG;
    float *alpha = l_run + kHG;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // blocks b, b+8, b+16, ... share an XCD (and its L2): give them consecutive work items,
    // so the head groups of one token range read the same tiles through one L2
    const int b = blockIdx.x;
    const int w = a.swizzle ? (b & 7) * (static_cast<int>(gridDim.x) >> 3) + (b >> 3) : b;
    const int HGn = (a.H + kHG - 1) / kHG;
    const int hg = w % HGn, split = w / HGn;
    const int h0 = hg * kHG;
    const int t0 = split * a.Ts;
    const int t_end = min(a.T, t0 + a.Ts);
    const int ntiles = (t_end - t0 + kTile - 1) / kTile;

    const auto rl = make_rsrc(a.lat, a.lat_bytes);
    const auto rr = make_rsrc(a.rot, a.rot_bytes);
    uint4 pre[kPre];
    auto load_tile = [&](int tb) {
#pragma unroll
        for (int i = 0; i < kPre; ++i) {
            const int c = tid + 256 * i;
            const int tok = c / kChunksPerRow, cc = c % kChunksPerRow;
            const int t = tb + tok;
            if (cc < kR / 8)
                pre[i] = buf_load16(rl, t < t_end ? static_cast<uint32_t>(t * a.ld_lat * 2 + cc * 16) : kOobOffset);
            else
                pre[i] = buf_load16(rr, t < t_end ? static_cast<uint32_t>(t * a.ld_rot * 2 + (cc - kR / 8) * 16)
                                                  : kOobOffset);
        }
    };
    load_tile(t0);

    // qa hi/lo of this block's heads into LDS (L2-resident: written by the Q launch)
    for (int c = tid; c < 2 * kHG * kChunksPerRow; c += 256) {
        const int hl = c / (kHG * kChunksPerRow), rem = c % (kHG * kChunksPerRow);
        const int hh = rem / kChunksPerRow, cc = rem % kChunksPerRow;
        const uint16_t *src = (hl ? a.qa_lo : a.qa_hi) + (h0 + hh) * kQaLd + cc * 8;
        // heads past H (last group of a head count that is not a multiple of 32) score 0
        *reinterpret_cast<uint4 *>(qa_s + (hl * kHG + hh) * kLdsRow + cc * 8) =
            h0 + hh < a.H ? *reinterpret_cast<const uint4 *>(src) : make_uint4(0u, 0u, 0u, 0u);
    }
    if (tid < kHG) {
        m_run[tid] = -INFINITY;
        l_run[tid] = 0.f;
    }

    f32x4_t cacc[2][8];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int n = 0; n < 8; ++n) cacc[m][n] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int r16 = lane & 15, q4 = lane >> 4;
    for (int it = 0; it < ntiles; ++it) {
        const int tb = t0 + it * kTile;
        __syncthreads();  // previous tile's LDS reads are done
#pragma unroll
        for (int i = 0; i < kPre; ++i) {
            const int c = tid + 256 * i;
            *reinterpret_cast<uint4 *>(lat_s + (c / kChunksPerRow) * kLdsRow + (c % kChunksPerRow) * 8) = pre[i];
        }
        __syncthreads();
        if (it + 1 < ntiles) load_tile(tb + kTile);

        // ---- scores: wave -> (head half mt, token half nt), K = 576 in 18 steps
        {
            const int mt = wave & 1, nt = wave >> 1;
            const uint16_t *ahi = qa_s + (mt * 16 + r16) * kLdsRow + q4 * 8;
            const uint16_t *alo = ahi + kHG * kLdsRow;
            const uint16_t *bp = lat_s + (nt * 16 + r16) * kLdsRow + q4 * 8;
            f32x4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 6
            for (int kk = 0; kk < kK / 32; ++kk) {
                const bf16x8 bv = *reinterpret_cast<const bf16x8 *>(bp + kk * 32);
                sacc = mfma_bf16(*reinterpret_cast<const bf16x8 *>(ahi + kk * 32), bv, sacc);
                sacc = mfma_bf16(*reinterpret_cast<const bf16x8 *>(alo + kk * 32), bv, sacc);
            }
            const int tok = nt * 16 + r16;
            const bool valid = tb + tok < t_end;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                s_s[(mt * 16 + q4 * 4 + i) * kSRow + tok] = valid ? sacc[i] * a.scale_log2 : -INFINITY;
        }
        __syncthreads();

        // ---- online softmax: 8 threads per head, 4 tokens each
        {
            const int hh = tid >> 3, q = tid & 7;
            float sv[4];
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sv[j] = s_s[hh * kSRow + q * 4 + j];
                mx = fmaxf(mx, sv[j]);
            }
            mx = fmaxf(mx, __shfl_xor(mx, 1, 8));
            mx = fmaxf(mx, __shfl_xor(mx, 2, 8));
            mx = fmaxf(mx, __shfl_xor(mx, 4, 8));
            const float mold = m_run[hh];
            const float mnew = fmaxf(mold, mx);  // finite: every tile holds a valid token
            float ps = 0.f;
            uint16_t *ph = p_s + hh * kPRow + q * 4;
            uint16_t *pl = ph + kHG * kPRow;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float p = exp2f(sv[j] - mnew);
                ps += p;
                split_bf16(p, ph[j], pl[j]);
            }
            ps += __shfl_xor(ps, 1, 8);
            ps += __shfl_xor(ps, 2, 8);
            ps += __shfl_xor(ps, 4, 8);
            if (q == 0) {
                const float al = exp2f(mold - mnew);
                alpha[hh] = al;
                l_run[hh] = l_run[hh] * al + ps;
                m_run[hh] = mnew;
            }
        }
        __syncthreads();

        // ---- ctx[32 x 512] += P @ tile: wave owns latent columns [128 wave, +128)
        {
            bf16x8 ph[2], pl[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                ph[m] = *reinterpret_cast<const bf16x8 *>(p_s + (m * 16 + r16) * kPRow + q4 * 8);
                pl[m] = *reinterpret_cast<const bf16x8 *>(p_s + (kHG + m * 16 + r16) * kPRow + q4 * 8);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float al = alpha[m * 16 + q4 * 4 + i];
#pragma unroll
                    for (int n = 0; n < 8; ++n) cacc[m][n][i] *= al;
                }
            }
            const uint16_t *col = lat_s + (q4 * 8) * kLdsRow + wave * 128 + r16;
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                uint16_t bv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) bv[i] = col[i * kLdsRow + n * 16];
                const bf16x8 bb = __builtin_bit_cast(bf16x8, bv);
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    cacc[m][n] = mfma_bf16(ph[m], bb, cacc[m][n]);
                    cacc[m][n] = mfma_bf16(pl[m], bb, cacc[m][n]);
                }
            }
        }
    }

    // ---- split record: unnormalised ctx, running max and sum
    float *part = a.part + (static_cast<int64_t>(split) * a.H + h0) * kPartLd;
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int n = 0; n < 8; ++n)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (h0 + m * 16 + q4 * 4 + i < a.H)
                    part[(m * 16 + q4 * 4 + i) * kPartLd + wave * 128 + n * 16 + r16] = cacc[m][n][i];
    if (tid < kHG && h0 + tid < a.H) {
        part[tid * kPartLd + kR] = m_run[tid];
        part[tid * kPartLd + kR + 1] = l_run[tid];
    }
}

// ------------------------------------------------------------------ M: merge + W_UV
struct MergeArgs {
    const float *part;
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

// grid: H * (V / 32); block (h, vq) merges head h and produces o[h][32 vq .. +32)
__global__ __launch_bounds__(256) void mla_merge_uv_kernel(MergeArgs a) {
    __shared__ float wsplit[kMaxSplits];
    __shared__ __align__(16) float ctx[2][kR];
    __shared__ float red[4];
    const int vqn = a.V / 32;
    const int h = blockIdx.x / vqn, vq = blockIdx.x % vqn;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *rec = a.part + static_cast<int64_t>(h) * kPartLd;
    const int64_t sstride = static_cast<int64_t>(a.H) * kPartLd;

    float mx = -INFINITY;
    for (int s = tid; s < a.NS; s += 256) mx = fmaxf(mx, rec[s * sstride + kR]);
    const float M = block_max256(mx, red);
    float ls = 0.f;
    for (int s = tid; s < a.NS; s += 256) {
        const float e = exp2f(rec[s * sstride + kR] - M);
        wsplit[s] = e;
        ls += e * rec[s * sstride + kR + 1];
    }
    const float inv_l = 1.0f / block_sum256(ls, red);  // block_sum256 synchronises wsplit

    {   // ctx = sum_s w_s ctx_s (two fixed halves of the splits, then their sum)
        const int r4 = tid & 127, half = tid >> 7;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s = half; s < a.NS; s += 2) {
            const float ws = wsplit[s];
            const float4 v = *reinterpret_cast<const float4 *>(rec + s * sstride + 4 * r4);
            acc.x = fmaf(ws, v.x, acc.x);
            acc.y = fmaf(ws, v.y, acc.y);
            acc.z = fmaf(ws, v.z, acc.z);
            acc.w = fmaf(ws, v.w, acc.w);
        }
        *reinterpret_cast<float4 *>(&ctx[half][4 * r4]) = acc;
    }
    __syncthreads();
    float c8[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c8[j] = (ctx[0][lane * 8 + j] + ctx[1][lane * 8 + j]) * inv_l;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int v = vq * 32 + wave * 8 + j;
        const uint4 w = *reinterpret_cast<const uint4 *>(a.w_uv + (static_cast<int64_t>(h) * a.V + v) * kR + lane * 8);
        const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
        float acc = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc = fmaf(__uint_as_float(wd[q] << 16), c8[2 * q], acc);
            acc = fmaf(__uint_as_float(wd[q] & 0xffff0000u), c8[2 * q + 1], acc);
        }
        acc = wave_sum_to_lane63(acc);
        if (lane == 63) {
            const int64_t o = static_cast<int64_t>(h) * a.ld_out + v;
            if (a.out_bf16)
                static_cast<uint16_t *>(a.out)[o] = f32_to_bf16(acc);
            else
                static_cast<float *>(a.out)[o] = acc;
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
    size_t qa_hi, qa_lo, part, total;
};

MlaWs mla_ws_layout(int64_t H, int64_t T) {
    int Ts, NS;
    mla_splits(std::max<int64_t>(T, 1), &Ts, &NS);
    MlaWs L{};
    auto up = [](size_t v) { return (v + 255) & ~size_t(255); };
    size_t o = 0;
    L.qa_hi = o, o += up(static_cast<size_t>(H) * kQaLd * 2);
    L.qa_lo = o, o += up(static_cast<size_t>(H) * kQaLd * 2);
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
    if (nope_dim <= 0 || nope_dim > 256 || v_dim <= 0 || v_dim % 32)
        return set_error(K3_ERR_SHAPE, "mla decode: nope=%lld must be in 1..256 and v=%lld a multiple of 32",
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
    static_assert(kAttnLds <= 160 * 1024, "attention LDS");
    rc = check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(&mla_attn_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kAttnLds)),
                   "mla decode: raise LDS limit");
    if (rc) return rc;
    mla_attn_kernel<<<dim3(static_cast<unsigned>(blocks)), 256, kAttnLds, st>>>(aa);
    rc = check_hip(hipGetLastError(), "mla decode: attention launch");
    if (rc) return rc;

    MergeArgs ma{part, static_cast<const uint16_t *>(w_uv), out, ld_out, static_cast<int>(H), NS,
                 static_cast<int>(v_dim), out_dtype == K3_BF16};
    mla_merge_uv_kernel<<<dim3(static_cast<unsigned>(H * (v_dim / 32))), 256, 0, st>>>(ma);
    return check_hip(hipGetLastError(), "mla decode: merge launch");
}
