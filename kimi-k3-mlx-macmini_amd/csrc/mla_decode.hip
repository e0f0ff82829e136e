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
//       block per CU); its wave pairs are independent streams over interleaved 16-token
//       steps, the two waves of a pair splitting the score contraction and the context
//       columns in halves.  Cache rows go HBM -> registers (MFMA operand layout, a ring of
//       buffers) -> a wave-private LDS copy for the transposed context operand.  Scores
//       S^T[16 tokens x 16 heads] come from bf16 MFMAs (v_mfma_f32_16x16x32_bf16) of the
//       rows against the hi and the lo half of qa; the pair adds its partials across one
//       barrier; a base-2 softmax turns them into P, split again into a bf16 hi/lo pair;
//       ctx^T += rows^T [P_hi; P_lo] on the same MFMA.  The streams merge in the block,
//       which writes its unnormalised (ctx, max, sum) record per head.
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

// Block: 16 heads x one split of Ts tokens, run by P pairs of waves.  Pair p is one
// flash-decoding stream over the 16-token steps p, p + P, p + 2P, ... of the split; its two
// waves split the score contraction and the context columns in halves:
//   wave j of the pair owns latent columns 256 j .. +256 and rope columns 32 j .. +32.
// Per step and wave:
//   load    its 9 column blocks of the 16 cache rows straight into MFMA operand layout
//           (lane (token r16, group q4) holds 8 consecutive columns of its row per block),
//           into a ring of RING register buffers, so RING - 1 steps are in flight
//   scores  partial S^T[token][head] = rows . qa over its columns (A = cache rows, B = qa hi
//           and lo, which stay in registers); the two partials meet through LDS across one
//           block barrier, and both waves add them in the same order, so both hold
//           identical scores.  Lane (head r16, q4) has tokens 4 q4 .. +3.
//   softmax per lane over its 4 tokens, the max reduced over the 4 lane rows; identical in
//           the two waves.  The max used for the exponentials moves only at the first step
//           of a pass; a later score above it by more than kSlack restarts the pass (of the
//           whole block, so every wave meets the same barriers).
//   ctx     ctx^T[col][head] += rows^T . P on the 16x16x32 bf16 MFMA with k-slots 0..3 =
//           P_hi and 4..7 = P_lo of the lane's own 4 tokens, so P needs no data movement;
//           the transposed rows come from a wave-private LDS copy via ds_read_b64_tr_b16,
//           duplicated into both k halves.  Lane (head r16, q4) accumulates ctx[head][256 j
//           + 16 n + 4 q4 .. +3] for its 16 column tiles n.
// The P streams meet once, in the final in-block merge.
constexpr int kStepT = 16;              // tokens per step
constexpr int kHalfK = 9;               // column blocks (of 32) per wave: 8 latent + 1 rope
constexpr int kHalfCols = kR / 2;       // latent columns per wave
constexpr int kCopyRow = kHalfCols + 8; // padded LDS row of the wave's copy (528 B)
constexpr size_t kCopyBytes = kStepT * kCopyRow * 2;  // 8448 B per wave and slot
constexpr float kSlack = 64.f;          // log2 headroom before the pass restarts
constexpr int kMaxPairs = 4;
constexpr int kTrBatch = 16;            // transposed reads issued ahead of their products
constexpr int kCsRow = kR + 4;          // padded LDS row of the merged context (floats)

template <int P>
constexpr size_t attn_lds_bytes() {  // two copy slots per wave; the merge reuses them
    return 2 * P * 2 * kCopyBytes;
}

template <int P, int RING>
__global__ __launch_bounds__(128 * P, 1) void mla_attn_kernel(AttnArgs a) {
    static_assert(P == 2 || P == 4, "pairs per block");
    static_assert(attn_lds_bytes<P>() >= static_cast<size_t>(P / 2) * 2 * 16 * 64 * 16, "merge buffers fit");
    static_assert(attn_lds_bytes<P>() >= static_cast<size_t>(kHG) * kCsRow * 4, "context staging fits");
    extern __shared__ uint4 smem[];
    __shared__ f32x4_t xs[P][2][2][64];  // partial scores: [pair][member][slot][lane]
    __shared__ int req[2];                         // restart requests by step parity (pass number)
    __shared__ float m_s[P][kHG], l_s[P][kHG];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pr = wave >> 1, j = wave & 1;
    const int r16 = lane & 15, q4 = lane >> 4;
    uint16_t *copy = reinterpret_cast<uint16_t *>(reinterpret_cast<char *>(smem) + wave * 2 * kCopyBytes);

    // blocks b, b+8, b+16, ... share an XCD (and its L2): give them consecutive work items,
    // so the head groups of one split read the same rows through one L2
    const int b = blockIdx.x;
    const int w = a.swizzle ? (b & 7) * (static_cast<int>(gridDim.x) >> 3) + (b >> 3) : b;
    const int HGn = (a.H + kHG - 1) / kHG;
    const int hg = w % HGn, split = w / HGn;
    const int h0 = hg * kHG;
    const int t_begin = split * a.Ts;
    const int t_end = min(a.T, t_begin + a.Ts);
    // every pair runs the block's step count (pair 0's): a step past a pair's tokens is all
    // masked and adds nothing, and the barriers of all waves stay matched
    const int nsteps = (t_end - t_begin + P * kStepT - 1) / (P * kStepT);

    if (tid < 2) req[tid] = 0;

    const auto rl = make_rsrc(a.lat, a.lat_bytes);
    const auto rr = make_rsrc(a.rot, a.rot_bytes);
    // Steps past nsteps and rows past T load zeros (out-of-range offsets), so every step
    // issues the same loads and the ring needs no guard; masked rows score -inf.
    auto load = [&](uint4(&buf)[kHalfK], int st) {
        const int t = t_begin + (st * P + pr) * kStepT + r16;
        const bool ok = t < t_end;
        const uint32_t ol = ok ? static_cast<uint32_t>(t) * a.lat_row_bytes + (j * kHalfCols + q4 * 8) * 2u : kOobOffset;
        const uint32_t orr = ok ? static_cast<uint32_t>(t) * a.rot_row_bytes + (j * 32 + q4 * 8) * 2u : kOobOffset;
#pragma unroll
        for (int k = 0; k < kHalfK - 1; ++k) buf[k] = buf_load16(rl, ol + k * 64u);
        buf[kHalfK - 1] = buf_load16(rr, orr);
    };
    // qa operands of head h0 + r16 over this wave's columns (heads past H load zeros),
    // issued before the ring so that waiting for a ring buffer also covers them
    bf16x8 qhi[kHalfK], qlo[kHalfK];
    {
        const uint32_t qbytes = static_cast<uint32_t>(a.H) * kQaLd * 2;
        const auto rqh = make_rsrc(a.qa_hi, qbytes), rql = make_rsrc(a.qa_lo, qbytes);
        const uint32_t qrow = h0 + r16 < a.H ? static_cast<uint32_t>((h0 + r16) * kQaLd + q4 * 8) * 2 : kOobOffset;
#pragma unroll
        for (int k = 0; k < kHalfK; ++k) {
            const uint32_t col = k < kHalfK - 1 ? j * kHalfCols + k * 32 : kR + j * 32;
            qhi[k] = __builtin_bit_cast(bf16x8, buf_load16(rqh, qrow + col * 2));
            qlo[k] = __builtin_bit_cast(bf16x8, buf_load16(rql, qrow + col * 2));
        }
    }
    uint4 buf[RING][kHalfK];

    __syncthreads();  // requests cleared

    f32x4_t cacc[kHalfCols / 16];
#pragma unroll
    for (int n = 0; n < kHalfCols / 16; ++n) cacc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_used = -INFINITY, l_run = 0.f;
    int pass = 0;  // restarts so far (block-uniform)

    // transposed-read source of this lane: row 4 q4 + r16 / 4, columns 4 (r16 % 4) .. +3
    typedef short s4_t __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s4_t *lds_s4;
    const uint16_t *tsrc = copy + (q4 * 4 + (r16 >> 2)) * kCopyRow + (r16 & 3) * 4;
    uint16_t *tdst = copy + r16 * kCopyRow + q4 * 8;

    // A step is split in two halves, software-pipelined one step apart: the front half of
    // step st + 1 (LDS copy, score products, refill of its buffer) is issued before the back
    // half of step st (exchange across the barrier, softmax, context products), so the
    // score products run on the matrix cores while the wave waits at the barrier and works
    // through the softmax.  The LDS copy has two slots (step parity): the front half writes
    // one while the back half reads the other.
    // A wave whose scores exceed its max by more than kSlack accumulates nothing from that
    // step on and posts a restart request; every wave sees it after the next barrier and
    // skips the rest of the pass too.
    bool again = false;
    f32x4_t mine = {0.f, 0.f, 0.f, 0.f};  // this wave's partial scores of the pending step
    auto front = [&](uint4(&bf)[kHalfK], int st) -> f32x4_t {
        // ---- partial scores over this wave's columns: hi and lo chains
        f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = s0;
#pragma unroll
        for (int k = 0; k < kHalfK; ++k) {
            const bf16x8 rk = __builtin_bit_cast(bf16x8, bf[k]);
            s0 = mfma_bf16(rk, qhi[k], s0);
            s1 = mfma_bf16(rk, qlo[k], s1);
        }
        // ---- latent columns of the rows -> the wave's LDS copy slot st & 1 (read last by
        // step st - 2, earlier in program order), then refill the buffer RING steps ahead
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        uint16_t *dst = tdst + (st & 1) * (kCopyBytes / 2);
#pragma unroll
        for (int k = 0; k < kHalfK - 1; ++k) *reinterpret_cast<uint4 *>(dst + k * 32) = bf[k];
        load(bf, st + RING);
        return s0 + s1;
    };
    auto back = [&](int st) {
        // ---- exchange the partials with the pair partner (slots alternate by step, so a
        // write never meets the partner's read of the previous step)
        const int slot = st & 1;
        xs[pr][j][slot][lane] = mine;
        __syncthreads();
        again = again || req[slot] > pass;  // requests of step st - 1 are visible here
        if (again) return;
        const f32x4_t other = xs[pr][j ^ 1][slot][lane];
        const f32x4_t sc = j == 0 ? mine + other : other + mine;

        // ---- softmax weights of this lane's tokens 4 q4 .. +3 of head r16
        const int tb = t_begin + (st * P + pr) * kStepT + q4 * 4;
        float s[4];
        float mt = -INFINITY;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            s[v] = tb + v < t_end ? sc[v] * a.scale_log2 : -INFINITY;
            mt = fmaxf(mt, s[v]);
        }
        mt = rows4_max(mt);  // -inf only for a step past the pair's tokens
        if (__any(mt > m_used + kSlack)) {
            m_used = fmaxf(m_used, mt);
            if (st != 0) {  // earlier steps used a smaller max: the block restarts
                req[slot ^ 1] = pass + 1;
                again = true;
                return;
            }
        }
        // p <= 2^kSlack; exponents below -126 flush to 0, far below the step's largest p.
        // Before the pair's first token the max is -inf and every p is 0.
        const float mref = m_used == -INFINITY ? 0.f : m_used;
        uint32_t pw[4];
#pragma unroll
        for (int v = 0; v < 4; v += 2) {
            const float p0 = __builtin_amdgcn_exp2f(s[v] - mref), p1 = __builtin_amdgcn_exp2f(s[v + 1] - mref);
            l_run += p0 + p1;
            const uint32_t hi = pack_bf16x2(p0, p1);
            pw[v / 2] = hi;
            pw[2 + v / 2] = pack_bf16x2(p0 - __uint_as_float(hi << 16), p1 - __uint_as_float(hi & 0xffff0000u));
        }
        const bf16x8 pb = __builtin_bit_cast(bf16x8, make_uint4(pw[0], pw[1], pw[2], pw[3]));

        // ---- ctx^T += rows^T . [P_hi; P_lo] over this wave's columns; all transposed
        // reads are issued before the first product, so their latencies overlap
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const uint16_t *src = tsrc + slot * (kCopyBytes / 2);
#pragma unroll
        for (int n0 = 0; n0 < kHalfCols / 16; n0 += kTrBatch) {
            s4_t t4[kTrBatch];
#pragma unroll
            for (int n = 0; n < kTrBatch; ++n)
                t4[n] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(src + (n0 + n) * 16));
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int n = 0; n < kTrBatch; ++n) {
                const bf16x8 ra = __builtin_bit_cast(bf16x8, __builtin_shufflevector(t4[n], t4[n], 0, 1, 2, 3, 0, 1, 2, 3));
                cacc[n0 + n] = mfma_bf16(ra, pb, cacc[n0 + n]);
            }
        }
    };
    // The max used by the exponentials (per head) is set by the first step of a pass and
    // only moves when a score exceeds it by more than kSlack (log2 units).  Then the block
    // restarts the pass from its first step, the triggering pair with its larger max, so the
    // accumulators are never rescaled inside the loop.  A restarted pass does not trigger
    // again on the steps before the trigger, so a block makes at most nsteps + 1 passes.
    // The trip loop runs whole trips of RING steps (steps past the split are all masked)
    // and has no other exit, so the waits at its top see the ring in steady-state order.
    for (;;) {
        // in buffer order (the trip loop waits for buffer r behind the loads of the others)
#pragma unroll
        for (int r = 0; r < RING; ++r) {
            load(buf[r], r);
            __builtin_amdgcn_sched_barrier(0);
        }
        again = false;
        mine = front(buf[0], 0);
        for (int st = 0; st < nsteps; st += RING) {
#pragma unroll
            for (int r = 0; r < RING; ++r) {
                const f32x4_t next = front(buf[(r + 1) % RING], st + r + 1);
                back(st + r);
                mine = next;
            }
        }
        __syncthreads();  // publishes a request made in the last step
        if (max(req[0], req[1]) <= pass) break;  // block-uniform
        ++pass;
#pragma unroll
        for (int n = 0; n < kHalfCols / 16; ++n) cacc[n] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        l_run = 0.f;
    }

    // ---- in-block merge of the P streams: common max, then a fixed pairwise tree
    const float l_tot = rows4_sum(l_run);
    if (j == 0 && q4 == 0) {
        m_s[pr][r16] = m_used;
        l_s[pr][r16] = l_tot;
    }
    __syncthreads();  // every stream is done with its LDS copies
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < P; ++v) M = fmaxf(M, m_s[v][r16]);  // finite: the split has a token
    const float f = m_used == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_used - M);
#pragma unroll
    for (int n = 0; n < kHalfCols / 16; ++n) cacc[n] *= f;
    float4 *xb = reinterpret_cast<float4 *>(smem);  // [P / 2][2][16][64] float4
#pragma unroll
    for (int half = P / 2; half >= 1; half /= 2) {
        if (pr >= half && pr < 2 * half) {
#pragma unroll
            for (int n = 0; n < kHalfCols / 16; ++n)
                xb[(((pr - half) * 2 + j) * 16 + n) * 64 + lane] = make_float4(cacc[n][0], cacc[n][1], cacc[n][2], cacc[n][3]);
        }
        __syncthreads();
        if (pr < half) {
#pragma unroll
            for (int n = 0; n < kHalfCols / 16; ++n) {
                const float4 o = xb[((pr * 2 + j) * 16 + n) * 64 + lane];
                cacc[n] += f32x4_t{o.x, o.y, o.z, o.w};
            }
        }
        __syncthreads();
    }
    // ---- the merged context goes out through LDS, so that each store of a wave writes
    // 1 KB of one record row (the merge buffers are free after the last barrier)
    float *cs = reinterpret_cast<float *>(smem);  // [16][kCsRow]
    if (pr == 0) {
#pragma unroll
        for (int n = 0; n < kHalfCols / 16; ++n)
            *reinterpret_cast<float4 *>(cs + r16 * kCsRow + j * kHalfCols + n * 16 + q4 * 4) =
                make_float4(cacc[n][0], cacc[n][1], cacc[n][2], cacc[n][3]);
        if (j == 0 && q4 == 0 && h0 + r16 < a.H) {
            float L = 0.f;
#pragma unroll
            for (int v = 0; v < P; ++v) {
                const float mv = m_s[v][r16];
                L += mv == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mv - M) * l_s[v][r16];
            }
            a.ml[static_cast<int64_t>(split) * a.H + h0 + r16] = make_float2(M, L);
        }
    }
    __syncthreads();
    float *rec = a.part + (static_cast<int64_t>(split) * a.H + h0) * kR;
    for (int f = tid; f < kHG * kR / 4; f += 128 * P) {
        const int row = f / (kR / 4), c4 = f % (kR / 4);
        if (h0 + row < a.H)
            *reinterpret_cast<float4 *>(rec + row * kR + c4 * 4) = *reinterpret_cast<const float4 *>(cs + row * kCsRow + c4 * 4);
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
constexpr int kPairs = 2;  // streams (wave pairs) per attention block: one wave per SIMD
constexpr int kRing = 2;   // register buffers per wave (deeper rings measured no faster)

// One attention block per CU: about 256 blocks of (head group, split); a split is a
// multiple of 16 kPairs tokens, so every step of every stream lies inside it.
void mla_splits(int64_t H, int64_t T, int *Ts, int *NS) {
    const int64_t hgn = cdiv(H, kHG);
    const int64_t want = std::max<int64_t>(1, 256 / hgn);
    int64_t ts = cdiv(T, want);
    ts = cdiv(ts, kStepT * kPairs) * kStepT * kPairs;
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
                               workspace, workspace_bytes, stream);
}

int k3::mla_decode_core(const void *q_nope, const void *q_rot, int64_t ld_q, int64_t ld_q_rot, int q_dtype,
                        const void *w_uk, const void *w_uv, const void *lat, int64_t ld_lat, const void *rot,
                        int64_t ld_rot, int64_t T, int64_t H, int64_t kv_lora_rank, int64_t rope_dim,
                        int64_t nope_dim, int64_t v_dim, float scale, void *out, int out_dtype, int64_t ld_out,
                        const float *gate, void *workspace, int64_t workspace_bytes, void *stream) {
    if (!q_nope || !q_rot || !w_uk || !w_uv || !lat || !rot || !out || !workspace)
        return set_error(K3_ERR_NULL, "mla decode: null pointer");
    if (q_dtype != K3_F32 && q_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "mla decode: q_dtype %d", q_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16)
        return set_error(K3_ERR_DTYPE, "mla decode: out_dtype %d", out_dtype);
    if (kv_lora_rank != kR || rope_dim != kRope)
        return set_error(K3_ERR_SHAPE, "mla decode: kv_lora_rank=%lld rope=%lld; the kernels take 512 and 64",
                         (long long)kv_lora_rank, (long long)rope_dim);
    if (H <= 0 || H > 4096) return set_error(K3_ERR_SHAPE, "mla decode: H=%lld must be in 1..4096", (long long)H);
    if (nope_dim <= 0 || nope_dim > 256 || v_dim <= 0 || v_dim > kMaxV)
        return set_error(K3_ERR_SHAPE, "mla decode: nope=%lld must be in 1..256 and v=%lld in 1..1024",
                         (long long)nope_dim, (long long)v_dim);
    if (T <= 0) return set_error(K3_ERR_SHAPE, "mla decode: empty cache (T=%lld)", (long long)T);
    if (ld_q < nope_dim || ld_q_rot < rope_dim || ld_lat < kR || ld_rot < kRope || ld_out < v_dim || ld_lat % 8 ||
        ld_rot % 8)
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
    aa.lat_row_bytes = static_cast<uint32_t>(ld_lat * 2);
    aa.rot_row_bytes = static_cast<uint32_t>(ld_rot * 2);
    aa.part = part;
    aa.ml = ml;
    aa.H = static_cast<int>(H);
    aa.T = static_cast<int>(T);
    aa.Ts = Ts;
    aa.NS = NS;
    aa.scale_log2 = scale * 1.4426950408889634f;
    const int blocks = NS * static_cast<int>(cdiv(H, kHG));
    aa.swizzle = blocks % 8 == 0;
    constexpr auto attn = &mla_attn_kernel<kPairs, kRing>;
    constexpr size_t lds = attn_lds_bytes<kPairs>();
    static const hipError_t lds_rc = hipFuncSetAttribute(reinterpret_cast<const void *>(attn),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                                         static_cast<int>(lds));  // may exceed the 64 KB default
    rc = check_hip(lds_rc, "mla decode: attention LDS size");
    if (rc) return rc;
    attn<<<dim3(static_cast<unsigned>(blocks)), 128 * kPairs, lds, st>>>(aa);
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
