// Routed MoE layer decode at batch 1 (router + top-k + routed experts + shared expert +
// weighted combine), three stream-ordered launches with no host synchronisation.
//
// Reference: LatentMoE.route / __call__ / shared_forward (air_llm/models/kimi_k3/moe.py:65-132,
// k3ref/layers.py:214-261).  The reference materialises the routing on the host
// (np_indices, moe.py:135-138) and loops over experts serially with an mx.eval per expert.
// Here the routing never leaves the GPU:
//
//   L1  router logits (bf16 [E, H] . x) and the shared expert's gate/up rows (bf16) with
//       its activation.  The router rows run in the first blocks; each router block counts
//       itself done on a workspace counter, and the last one computes softmax / sigmoid,
//       the exact top-k (ties to the lower expert index), the router records and the
//       selected experts' weight pointers -- while the shared stream is still running.
//   L2  the shared expert's down rows (bf16 [H, Is] . shared act) in the first blocks, which
//       need no routing, then the routed gate/up row pairs of the k selected experts (MXFP4,
//       through the device pointer table, so every expert stays resident and each selected
//       expert's bytes are read once) with their activation.
//   L3  per block, one selected expert and 4*RW down rows (RW per wave): each lane holds the
//       act values of its pieces of the row in registers and the wave reduces its rows; the
//       row totals go to the workspace, and the last of the k blocks of a row range to
//       finish (an arrival counter per range) combines y = shared + sum_j w_j * down_j in
//       slot order.
//
// K3's latent layer (k3_moe_latent_layer_decode) runs the same launches in a latent mode:
// L1 also computes h = bf16(W_down x), L2 and L3 read and write the latent width, L3 writes
// the routed sum ylat, and a fourth launch (the dense row kernel of dense_rows.h) takes the
// rows of W_up against rmsnorm(ylat) * norm and adds the shared output.
//
// Every kernel issues its activation loads, then its whole weight stream, before it stages
// anything into LDS or registers it consumes, and stages with unconditional stores, so the
// in-order vmcnt waits never hold the staging behind the weight stream.
#include <algorithm>
#include <atomic>

#include "dense_rows.h"
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
    uint32_t *counter;   // [0] router blocks done (L1), [1 + r] blocks of L3 row range r
                         // done; every launch returns them to 0
    float *yrow;         // [k][Hr] per-slot down-row totals (L3)
    void *h;             // [Hr] latent state (latent layer): bf16 for a bf16 x, fp32 for an fp32 x
    float *ylat;         // [Hr] routed sum in latent space (latent layer)
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
    int l1_router_blocks;          // L1: blocks [0, l1_router_blocks) do router rows
    int l2_shared_blocks;          // L2: blocks [0, l2_shared_blocks) do shared down rows
    // K3's latent wrapper (moe.py:116,129-130); lat_down == null: the plain layer
    int Hr;                        // width the routed experts read and write (H, or the latent width)
    const uint16_t *lat_down;      // [Hr, H] bf16: h = x W_down^T (bf16 for a bf16 x, as the reference)
    const uint16_t *lat_up;        // [H, Hr] bf16
    const float *lat_norm;         // [Hr] KimiRMSNorm weight
    float eps;
    int l1_latent_blocks;          // L1: the next blocks do latent down rows (4 per block)
    int l3_ranges;                 // L3: row ranges (one arrival counter each)
};

constexpr int kMaxTopK = 16;
constexpr int kMaxExperts = 1024;
// Arrival counters at the head of the workspace: [0] for L1's router blocks, [1 + r] for the
// blocks of L3's row range r
constexpr size_t kCounterBytes = 4096;
constexpr int kSharedDownRows = 2;  // shared down rows per wave (L2)
// shared down rows per wave for CHI chunks per lane: one row past 8 chunks (wide shared
// experts), so the fp32 activation and the rows stay in registers
constexpr int shared_down_rows(int chi) { return chi > 8 ? 1 : kSharedDownRows; }
// routed (gate, up) row pairs per wave (L2): one keeps L2 at 62-70 VGPRs (seven or eight
// waves per SIMD); two: 384-expert layer 56.6 -> 57.7 us, K3's 126.8 -> 128.3 us; three or
// four: 59.4 / 59.7 us
constexpr int kRoutedPairs = 1;

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

// Activation row staging in two halves: x_load issues XREG 16-byte loads per thread
// (out-of-range chunks read zeros), x_store writes them all; callers issue their weight
// stream between the two.  `swz` picks the swizzled MXFP4 group order (XTile) or the plain
// chunk order of the bf16 rows.
template <int XREG>
__device__ __forceinline__ void x_load(uint4 (&xr)[XREG], const void *x, int nchunks) {
    const auto rx = make_rsrc(x, static_cast<uint32_t>(nchunks * 16));
#pragma unroll
    for (int k = 0; k < XREG; ++k) {
        const int c = threadIdx.x + 256 * k;
        xr[k] = buf_load16(rx, c < nchunks ? static_cast<uint32_t>(c) * 16u : kOobOffset);
    }
}
template <typename XT, int XREG, bool SWZ>
__device__ __forceinline__ void x_store(uint4 *xl, const uint4 (&xr)[XREG]) {
    constexpr int CPG = XTile<XT>::kChunks;
#pragma unroll
    for (int k = 0; k < XREG; ++k) {
        const int c = threadIdx.x + 256 * k;
        xl[SWZ ? XTile<XT>::slot(c / CPG, c % CPG) : c] = xr[k];
    }
}
template <typename XT>
constexpr int x_regs() { return sizeof(XT) == 2 ? 4 : 8; }  // H <= 8192

// ------------------------------------------------------------------ routing (one block)
// softmax:       scores = softmax(logits), selection on scores
// sigmoid_bias:  scores = sigmoid(logits), selection on scores + bias, weights from scores
// weights: optional renormalisation by (sum + 1e-20), then * scaling   (moe.py:65-76)
// Top-k is exact and deterministic with ties to the lower expert index: the order is the
// strict total order on (selection score, -index), with NaN scores ranked as -inf, as one
// 64-bit key per expert.  No sequential selection rounds over the experts: a lower bound on
// the k-th largest key from a small sample picks out a few candidates, and the candidates
// are ranked in parallel (each lane of a wave counts the larger keys among the wave's 64,
// each key broadcast from its lane through v_readlane), in a merge tree of 64-wide groups
// whose best k go on, until one group remains.
// 64-bit order key of (selection score, expert): larger key = ranks first.  High word: the
// float's bits mapped monotonically to unsigned (NaN mapped as -inf); low word: the
// complement of the expert index, so ties go to the lower index.  Every live expert's key
// is nonzero; 0 marks an empty slot.
__device__ __forceinline__ uint64_t order_key(float v, int e) {
    if (v != v) v = -INFINITY;
    const uint32_t b = __float_as_uint(v);
    const uint32_t mono = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (static_cast<uint64_t>(mono) << 32) | (0xffffffffu - static_cast<uint32_t>(e));
}
__device__ __forceinline__ int key_expert(uint64_t k) { return static_cast<int>(0xffffffffu - static_cast<uint32_t>(k)); }

// Lane l's 64-bit key, broadcast (SGPR pair); l is wave-uniform.
__device__ __forceinline__ uint64_t readlane_key(uint64_t v, int l) {
    return (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), l))) << 32) |
           static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), l));
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_key(uint64_t v) {
    const uint32_t lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v)), CTRL, 0xf, 0xf, false);
    const uint32_t hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(v >> 32), CTRL, 0xf, 0xf, false);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint64_t max_key(uint64_t a, uint64_t b) { return a > b ? a : b; }
// Largest key of each 16-lane row, in every lane of the row (DPP only, as wave_max_all).
__device__ __forceinline__ uint64_t row_max_key(uint64_t v) {
    v = max_key(v, dpp_key<0xb1>(v));
    v = max_key(v, dpp_key<0x4e>(v));
    v = max_key(v, dpp_key<0x141>(v));
    return max_key(v, dpp_key<0x140>(v));
}
// Number of lanes j < n (n wave-uniform, at most 64) whose key is larger than this lane's,
// in batches of 16 lanes (the reads of a batch ahead of its compares); lanes from n up to the
// end of the last batch must hold keys no larger than any counted lane's (0 for an empty slot).
__device__ __forceinline__ int wave_rank_upto(uint64_t key, int n) {
    const int hi = static_cast<int>(key >> 32), lo = static_cast<int>(key);
    int rank = 0;
#pragma unroll
    for (int j0 = 0; j0 < 64; j0 += 16) {
        if (j0 >= n) break;  // uniform
        uint32_t h[16], w[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            h[j] = __builtin_amdgcn_readlane(hi, j0 + j);
            w[j] = __builtin_amdgcn_readlane(lo, j0 + j);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 16; ++j) rank += ((static_cast<uint64_t>(h[j]) << 32) | w[j]) > key;
    }
    return rank;
}
// The same for a wave whose lane j holds expert e0 + j: the low word of
// lane j's key is known without a read (order_key), so only the high word is broadcast.  A
// lane past the last expert holds high word 0, below every live key.
__device__ __forceinline__ int wave_rank_experts(uint64_t key, int e0) {
    const int hi = static_cast<int>(key >> 32);
    int rank = 0;
#pragma unroll
    for (int j0 = 0; j0 < 64; j0 += 16) {
        uint32_t h[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) h[j] = __builtin_amdgcn_readlane(hi, j0 + j);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 16; ++j)
            rank += ((static_cast<uint64_t>(h[j]) << 32) | (0xffffffffu - static_cast<uint32_t>(e0 + j0 + j))) > key;
    }
    return rank;
}
// A wave's best k entries to out_k/out_v[0, k): the live lane of rank r < k writes slot r
// (live keys are distinct, so their ranks are 0 .. n_live - 1) and slots from n_live to k
// get key 0, which ranks below every live key.
__device__ __forceinline__ void emit_best(uint64_t key, float v, int rank, bool live, int k, uint64_t *out_k,
                                          float *out_v) {
    const int lane = threadIdx.x & 63;
    const int n_live = __builtin_popcountll(__builtin_amdgcn_ballot_w64(live));
    if (live && rank < k) {
        out_k[rank] = key;
        out_v[rank] = v;
    }
    if (lane >= n_live && lane < k) out_k[lane] = 0;
}

// Called by all 256 threads of the last router block; logits are read with agent-coherent
// loads (written by other blocks, possibly on other XCDs, in this launch).
//
// Selection values: sigmoid(logit) + bias for sigmoid_bias; for softmax the logit itself,
// since the probability is a strictly increasing function of it (the fp64 probabilities
// order exactly as the logits; fp32 ones may round distinct logits to one value).  A NaN
// logit makes every softmax probability NaN; then all scores tie and the k lowest indices
// are selected, as for any all-NaN score row.
//
// Steps (each thread holds experts t + 256 m):
//   1. keys; per-wave softmax partials (max, sum of exp); a sample of four keys per
//      64-expert group: the largest key of each of its 16-lane rows (DPP row maxima), when
//      the samples number at least k;
//   2. theta = the k-th largest sample: the samples are keys, so at least k keys are at
//      least theta and every key of the top k is; only the k rows whose maximum reaches
//      theta hold such keys, so these survivors number at most 16 k (typically 9 to 20);
//      they are collected in LDS;
//   3. the survivors, or without a sample every key, go through the ranking merge tree
//      until one group of at most 64 is left, whose ranks are the selection order.
// No wave stores to memory before it has waited for its table loads: vmcnt counts stores as
// well as loads, so a store issued before that wait would hold it for a store round trip.
__device__ void route_block(const LayerArgs &a) {
    constexpr int kPer = kMaxExperts / 256;  // experts per thread: e = t + 256 * m
    constexpr int kMaxCand = kMaxExperts / 64 * kMaxTopK;
    __shared__ uint64_t cand_k[2][kMaxCand];
    __shared__ float cand_v[2][kMaxCand];
    __shared__ uint64_t samp_s[4 * (kMaxExperts / 64)];
    __shared__ float stat_s[2][4];
    __shared__ uint32_t nsurv_s;
    __shared__ uint8_t slot_s[kMaxExperts];  // selection slot of expert e; 0xff: not selected
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const bool soft = a.route_kind == K3_ROUTE_SOFTMAX;
    const bool biased = a.route_kind == K3_ROUTE_SIGMOID_BIAS && a.router_bias;
    float l[kPer], bias[kPer];
#pragma unroll
    for (int m = 0; m < kPer; ++m) {
        const int e = t + 256 * m;
        l[m] = e < a.E ? __hip_atomic_load(a.ws.logits + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -INFINITY;
    }
    // the bias and the 6 table pointers of this thread's experts are loaded alongside the
    // logits, so no dependent load waits later
    {
        const auto rb = make_rsrc(a.router_bias, biased ? static_cast<uint32_t>(a.E) * 4u : 0u);
#pragma unroll
        for (int m = 0; m < kPer; ++m) {
            const int e = t + 256 * m;
            bias[m] = __uint_as_float(buf_load4(rb, e < a.E ? static_cast<uint32_t>(e) * 4u : kOobOffset));
        }
    }
    uint4 tab[kPer][3];
    {
        const auto rt = make_rsrc(a.table, a.table ? static_cast<uint32_t>(a.E) * 48u : 0u);
#pragma unroll
        for (int m = 0; m < kPer; ++m) {
            const int e = t + 256 * m;
#pragma unroll
            for (int q = 0; q < 3; ++q) tab[m][q] = buf_load16(rt, e < a.E ? static_cast<uint32_t>(e) * 48u + q * 16u : kOobOffset);
        }
    }
    // 1. keys (v: the value a candidate carries, the logit for softmax, else the score)
    uint64_t key[kPer];
    float v[kPer], sel[kPer];
#pragma unroll
    for (int m = 0; m < kPer; ++m) {
        const int e = t + 256 * m;
        if (soft) {
            v[m] = sel[m] = l[m];
        } else {
            v[m] = 1.0f / (1.0f + expf(-l[m]));
            sel[m] = biased ? v[m] + bias[m] : v[m];
        }
        key[m] = e < a.E ? order_key(sel[m], e) : 0;
        slot_s[e] = 0xff;
    }
    if (t == 0) nsurv_s = 0;
    if (soft) {  // per-wave max and sum of exp(logit - max); a NaN logit makes the sum NaN
        float mx = -INFINITY;
#pragma unroll
        for (int m = 0; m < kPer; ++m) mx = fmaxf(mx, l[m]);
        mx = wave_max_all(mx);
        float sum = 0.f;
#pragma unroll
        for (int m = 0; m < kPer; ++m)
            if (t + 256 * m < a.E) sum += l[m] != l[m] ? l[m] : (mx == -INFINITY ? 0.f : expf(l[m] - mx));
        sum = wave_sum_all(sum);
        if (lane == 0) {
            stat_s[0][wave] = mx;
            stat_s[1][wave] = sum;
        }
    }
    const int g1 = (a.E + 63) / 64;  // 64-expert groups
    const int ns = 4 * g1;           // samples: the largest key of each 16-lane row of a group
    const bool sampled = ns >= a.k;
    if (sampled) {
#pragma unroll
        for (int m = 0; m < kPer; ++m) {
            const int g = 4 * m + wave;
            if (g < g1) {  // uniform per wave
                const uint64_t rm = row_max_key(key[m]);
                if ((lane & 15) == 0) samp_s[4 * g + (lane >> 4)] = rm;
            }
        }
    }
    __syncthreads();
    // softmax statistics from the per-wave partials; every probability uses the same max
    float M = 0.f, S = 1.f;
    if (soft) {
        M = fmaxf(fmaxf(stat_s[0][0], stat_s[0][1]), fmaxf(stat_s[0][2], stat_s[0][3]));
        S = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) S += stat_s[1][w] == 0.f ? 0.f : stat_s[1][w] * expf(stat_s[0][w] - M);
    }
    const bool nan_route = soft && !(S > 0.f);  // a NaN or infinite logit: every probability NaN
    int n = 0, buf = 0;
    if (sampled) {
        // 2. theta (every wave computes it) and the survivors, one LDS atomic per wave
        const uint64_t ks = lane < ns ? samp_s[lane] : 0;
        const int rs = wave_rank_upto(ks, ns);
        const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < ns && rs == a.k - 1);
        const uint64_t theta = hit ? readlane_key(ks, __builtin_ctzll(hit)) : 0;
        bool sv[kPer];
        uint64_t mask[kPer];
        uint32_t cnt = 0;
#pragma unroll
        for (int m = 0; m < kPer; ++m) {
            sv[m] = key[m] != 0 && key[m] >= theta;
            mask[m] = __builtin_amdgcn_ballot_w64(sv[m]);
            cnt += static_cast<uint32_t>(__builtin_popcountll(mask[m]));
        }
        uint32_t base = 0;
        if (cnt) {  // uniform
            if (lane == 0) base = atomicAdd(&nsurv_s, cnt);
            base = __builtin_amdgcn_readfirstlane(base);
        }
#pragma unroll
        for (int m = 0; m < kPer; ++m) {
            const uint32_t pos = base + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask[m] >> 32),
                                                                  __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask[m]), 0u));
            if (sv[m] && pos < kMaxCand) {
                cand_k[0][pos] = key[m];
                cand_v[0][pos] = v[m];
            }
            base += static_cast<uint32_t>(__builtin_popcountll(mask[m]));
        }
        __syncthreads();
        n = static_cast<int>(nsurv_s);
    }
    if (!sampled || n > kMaxCand) {
        // 3'. every key: each wave ranks its 64 experts of round m (experts 256 m + 64 wave + lane)
#pragma unroll
        for (int m = 0; m < kPer; ++m) {
            const int g = 4 * m + wave;
            if (g < g1) {  // uniform per wave
                const int rank = wave_rank_experts(key[m], 64 * g);
                emit_best(key[m], v[m], rank, key[m] != 0, a.k, cand_k[0] + g * a.k, cand_v[0] + g * a.k);
            }
        }
        n = g1 * a.k;
        __syncthreads();
    }
    // 3. ranking levels while more than one group of 64 candidates is left
    while (n > 64) {
        const int ng = (n + 63) / 64;
        for (int g = wave; g < ng; g += 4) {
            const int c = g * 64 + lane;
            const uint64_t kc = c < n ? cand_k[buf][c] : 0;
            const float vc = c < n ? cand_v[buf][c] : 0.f;
            emit_best(kc, vc, wave_rank_upto(kc, 64), kc != 0, a.k, cand_k[buf ^ 1] + g * a.k, cand_v[buf ^ 1] + g * a.k);
        }
        buf ^= 1;
        n = ng * a.k;
        __syncthreads();
    }
    // the router records of this thread's experts, after the wave's wait for its table loads
    auto store_records = [&]() {
#pragma unroll
        for (int m = 0; m < kPer; ++m)
#pragma unroll
            for (int q = 0; q < 3; ++q) asm volatile("" ::"v"(tab[m][q].x), "v"(tab[m][q].w));
#pragma unroll
        for (int m = 0; m < kPer; ++m) {
            const int e = t + 256 * m;
            if (e < a.E) {
                const float sc = soft ? expf(l[m] - M) / S : v[m];
                a.ws.scores[e] = sc;
                a.ws.corrected[e] = soft ? sc : sel[m];
            }
        }
    };
    // the last group (wave 0): the lane of rank r < k holds the r-th selected expert; waves
    // 1-3 store their records meanwhile
    bool chosen = false;
    int rank = 0, esel = 0;
    float wsel = 0.f;
    if (wave == 0) {
        const uint64_t kc = lane < n ? cand_k[buf][lane] : 0;
        const float vc = lane < n ? cand_v[buf][lane] : 0.f;
        float sc;
        if (nan_route) {
            rank = esel = lane;
            chosen = lane < a.k;
            sc = __int_as_float(0x7fc00000);
        } else {
            rank = wave_rank_upto(kc, n);
            chosen = kc != 0 && rank < a.k;
            esel = key_expert(kc);
            sc = soft ? expf(vc - M) / S : vc;
        }
        const float wsum = wave_sum_all(chosen ? sc : 0.f);
        const float norm = (a.renorm && a.k > 1) ? 1.0f / (wsum + 1e-20f) : 1.0f;
        wsel = sc * norm * a.scaling;
        if (chosen) slot_s[esel] = static_cast<uint8_t>(rank);
    } else {
        store_records();
    }
    if (a.table) {  // the owner of each selected expert writes its pointers
        __syncthreads();
#pragma unroll
        for (int m = 0; m < kPer; ++m) {
            const int e = t + 256 * m;
            if (256 * m >= a.E) break;  // uniform: no expert of this or later rounds
            const int r = slot_s[e];
            if (r != 0xff) {
                uint4 *dst = reinterpret_cast<uint4 *>(a.ws.sel_ptrs + r * 6);
                dst[0] = tab[m][0];
                dst[1] = tab[m][1];
                dst[2] = tab[m][2];
            }
        }
    }
    if (chosen) {
        a.ws.topk_idx[rank] = esel;
        a.ws.topk_w[rank] = wsel;
    }
    if (wave == 0) store_records();
}

// ------------------------------------------------------------------ batched selection
// One block per token: route_block on router logits computed elsewhere (the prefill path
// takes them from a GEMM over all tokens), with the token's records at its row of each
// output array.  No pointer table: a.table is null.
__global__ __launch_bounds__(256) void topk_kernel(LayerArgs a, int64_t ld_logits) {
    const int64_t t = blockIdx.x;
    LayerArgs b = a;
    b.ws.logits = a.ws.logits + t * ld_logits;
    b.ws.scores = a.ws.scores + t * a.E;
    b.ws.corrected = a.ws.corrected + t * a.E;
    b.ws.topk_idx = a.ws.topk_idx + t * a.k;
    b.ws.topk_w = a.ws.topk_w + t * a.k;
    route_block(b);
}

// ------------------------------------------------------------------ L1
// CHH: bf16 chunks (8 elements) per lane over H.  UP_DELAY: the shared blocks issue their up
// rows' loads ~1.6 us after their gate rows' (a template parameter: a runtime branch between
// the two load orders measured as slow as no delay at all).
template <typename XT, int CHH, bool UP_DELAY>
__global__ __launch_bounds__(256) void layer_l1(LayerArgs a) {
    extern __shared__ uint4 smem[];
    __shared__ uint32_t last_s;
    constexpr int XREG = x_regs<XT>();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const uint32_t row_bytes = static_cast<uint32_t>(a.H) * 2u;
    const int nch = a.H >> 3;
    const int xchunks = a.H * static_cast<int>(sizeof(XT)) / 16;
    uint4 xr[XREG];
    x_load<XREG>(xr, a.x, xchunks);
    if (static_cast<int>(blockIdx.x) < a.l1_router_blocks) {
        const int e = blockIdx.x * 4 + wave;
        const auto r = make_rsrc(a.router_w, static_cast<uint32_t>(a.E) * row_bytes);
        uint4 w[CHH];
#pragma unroll
        for (int u = 0; u < CHH; ++u) {
            const int c = u * 64 + lane;
            w[u] = buf_load16_nt(r, (e < a.E && c < nch) ? static_cast<uint32_t>(e) * row_bytes + c * 16u : kOobOffset);
        }
        x_store<XT, XREG, false>(smem, xr);
        __syncthreads();
        float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
        for (int u = 0; u < CHH; ++u) {
            const int c = u * 64 + lane;
            if (c < nch) {
                if (u & 1)
                    acc1 = dot_chunk<XT>(w[u], smem, c, acc1);
                else
                    acc0 = dot_chunk<XT>(w[u], smem, c, acc0);
            }
        }
        const float tot = wave_sum_to_lane63(acc0 + acc1);
        if (lane == 63 && e < a.E)
            __hip_atomic_store(a.ws.logits + e, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);  // each wave's logit store is complete ...
        __syncthreads();
        if (threadIdx.x == 0) {         // ... before the block counts itself done
            // The logits are agent-scope atomic stores (written through to the coherence
            // point) and every wave has waited for their completion above, so the count is
            // made after they are visible device-wide; the block that brings it to the number
            // of router blocks runs an agent-scope acquire and routes on every block's
            // logits.  (A release RMW per block would add an L2 writeback per router block:
            // measured 62 -> 95 us per layer when the L3 blocks did the same.)  The counter is
            // zero at the start of a call: that block returns it to zero, and L2 of every
            // call zeroes it as well (a workspace that started with garbage there routes
            // correctly from its second call on).
            const uint32_t old = __hip_atomic_fetch_add(a.ws.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last_s = old + 1 == static_cast<uint32_t>(a.l1_router_blocks);
            if (last_s) {
                __hip_atomic_store(a.ws.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            }
        }
        __syncthreads();
        if (last_s) route_block(a);
    } else if (static_cast<int>(blockIdx.x) < a.l1_router_blocks + a.l1_latent_blocks) {
        // latent down rows: h[l] = W_down[l] . x, rounded to bf16 for a bf16 x (the reference's
        // bf16 matmul) and kept in fp32 for an fp32 x (its bf16 x fp32 promotion)
        const int l = (blockIdx.x - a.l1_router_blocks) * 4 + wave;
        const auto r = make_rsrc(a.lat_down, static_cast<uint32_t>(a.Hr) * row_bytes);
        uint4 w[CHH];
#pragma unroll
        for (int u = 0; u < CHH; ++u) {
            const int c = u * 64 + lane;
            w[u] = buf_load16_nt(r, (l < a.Hr && c < nch) ? static_cast<uint32_t>(l) * row_bytes + c * 16u : kOobOffset);
        }
        x_store<XT, XREG, false>(smem, xr);
        __syncthreads();
        float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
        for (int u = 0; u < CHH; ++u) {
            const int c = u * 64 + lane;
            if (c < nch) {
                if (u & 1)
                    acc1 = dot_chunk<XT>(w[u], smem, c, acc1);
                else
                    acc0 = dot_chunk<XT>(w[u], smem, c, acc0);
            }
        }
        const float tot = wave_sum_to_lane63(acc0 + acc1);
        if (lane == 63 && l < a.Hr) {
            if constexpr (sizeof(XT) == 2)
                static_cast<uint16_t *>(a.ws.h)[l] = f32_to_bf16(tot);
            else
                static_cast<float *>(a.ws.h)[l] = tot;
        }
    } else {
        // ~0.2 us head start for the router rows' loads (issued by the first blocks): the
        // router blocks then finish early and the routing block runs under this stream
        __builtin_amdgcn_s_sleep(8);
        const int i = (blockIdx.x - a.l1_router_blocks - a.l1_latent_blocks) * 4 + wave;
        const bool v = i < a.Is;
        const auto rg = make_rsrc(a.sh_gate, static_cast<uint32_t>(a.Is) * row_bytes);
        const auto ru = make_rsrc(a.sh_up, static_cast<uint32_t>(a.Is) * row_bytes);
        uint4 wg[CHH], wu[CHH];
        if constexpr (UP_DELAY) {
            // The whole grid is resident at once, so router blocks share their CUs with these
            // blocks, and a CU delivers about 10 bytes per clock to all its blocks together:
            // with the up rows' loads held back the router rows get a larger share of their
            // CU, the last router block finishes earlier and the routing runs under this
            // stream (the gate rows keep every CU busy meanwhile).
#pragma unroll
            for (int u = 0; u < CHH; ++u) {
                const int c = u * 64 + lane;
                wg[u] = buf_load16_nt(rg, (v && c < nch) ? static_cast<uint32_t>(i) * row_bytes + c * 16u : kOobOffset);
            }
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_sleep(60);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < CHH; ++u) {
                const int c = u * 64 + lane;
                wu[u] = buf_load16_nt(ru, (v && c < nch) ? static_cast<uint32_t>(i) * row_bytes + c * 16u : kOobOffset);
            }
        } else {
#pragma unroll
            for (int u = 0; u < CHH; ++u) {
                const int c = u * 64 + lane;
                const uint32_t off = (v && c < nch) ? static_cast<uint32_t>(i) * row_bytes + c * 16u : kOobOffset;
                wg[u] = buf_load16_nt(rg, off);
                wu[u] = buf_load16_nt(ru, off);
            }
        }
        x_store<XT, XREG, false>(smem, xr);
        __syncthreads();
        float ag = 0.f, au = 0.f;
#pragma unroll
        for (int u = 0; u < CHH; ++u) {
            const int c = u * 64 + lane;
            if (c < nch) {
                ag = dot_chunk<XT>(wg[u], smem, c, ag);
                au = dot_chunk<XT>(wu[u], smem, c, au);
            }
        }
        ag = wave_sum_to_lane63(ag);
        au = wave_sum_to_lane63(au);
        if (lane == 63 && v) a.ws.shared_act[i] = act_fn(ag, au, a.act_kind, a.beta, a.lbeta);
    }
}

// ------------------------------------------------------------------ L2
// GA: MXFP4 groups per lane over H.  CHI: bf16 chunks per lane over Is.
template <typename XT, int GA, int CHI>
__global__ __launch_bounds__(256) void layer_l2(LayerArgs a) {
    extern __shared__ uint4 smem[];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    // L1 is complete and L3 has not started: zero L1's counter and L3's range counters, so
    // each call starts from zeros whatever the counter bytes held before
    if (blockIdx.x == 0)
        for (int c = threadIdx.x; c < 1 + a.l3_ranges; c += 256) a.ws.counter[c] = 0u;
    if (static_cast<int>(blockIdx.x) < a.l2_shared_blocks) {
        // shared down: kSharedDownRows bf16 rows [H, Is] per wave against the fp32 shared act,
        // which each lane holds in registers for its own chunks (L2-resident after the first
        // waves)
        constexpr int SDR = shared_down_rows(CHI);
        const int n0 = (blockIdx.x * 4 + wave) * SDR;
        const uint32_t row_bytes = static_cast<uint32_t>(a.Is) * 2u;
        const int nch = a.Is >> 3;
        const auto ra = make_rsrc(a.ws.shared_act, static_cast<uint32_t>(a.Is) * 4u);
        float4 av[CHI][2];
#pragma unroll
        for (int u = 0; u < CHI; ++u) {
            const int c = u * 64 + lane;
            const bool ok = c < nch;
            av[u][0] = __builtin_bit_cast(float4, buf_load16(ra, ok ? c * 32u : kOobOffset));
            av[u][1] = __builtin_bit_cast(float4, buf_load16(ra, ok ? c * 32u + 16u : kOobOffset));
        }
        const auto rr = make_rsrc(a.sh_down, static_cast<uint32_t>(a.H) * row_bytes);
        uint4 w[SDR][CHI];
#pragma unroll
        for (int r = 0; r < SDR; ++r)
#pragma unroll
            for (int u = 0; u < CHI; ++u) {
                const int c = u * 64 + lane, n = n0 + r;
                w[r][u] = buf_load16_nt(rr, (n < a.H && c < nch) ? static_cast<uint32_t>(n) * row_bytes + c * 16u
                                                                : kOobOffset);
            }
#pragma unroll
        for (int r = 0; r < SDR; ++r) {
            float acc = 0.f;
#pragma unroll
            for (int u = 0; u < CHI; ++u) acc = dot8(w[r][u], av[u][0], av[u][1], acc);
            const float t = wave_sum_to_lane63(acc);
            if (lane == 63 && n0 + r < a.H) a.ws.yshared[n0 + r] = t;
        }
        return;
    }
    // routed gate/up: kRoutedPairs (slot j, row i) pairs per wave, over the routed input
    // (x, or the latent state h, which has x's dtype)
    constexpr int CPGX = XTile<XT>::kChunks;
    constexpr int XREG = x_regs<XT>();
    const int GH = a.Hr >> 5;
    const uint32_t rowA = static_cast<uint32_t>(a.Hr >> 1);
    uint4 xr[XREG];
    x_load<XREG>(xr, a.lat_down ? static_cast<const void *>(a.ws.h) : a.x, GH * CPGX);
    uint4 wg[kRoutedPairs][GA], wu[kRoutedPairs][GA];
    uint32_t sg[kRoutedPairs][GA], su[kRoutedPairs][GA];
    int jj[kRoutedPairs], ii[kRoutedPairs];
    bool vv[kRoutedPairs];
#pragma unroll
    for (int p = 0; p < kRoutedPairs; ++p) {
        const int pair = ((blockIdx.x - a.l2_shared_blocks) * 4 + wave) * kRoutedPairs + p;
        const int j = pair / a.I, i = pair % a.I;
        const bool v = j < a.k;
        jj[p] = j, ii[p] = i, vv[p] = v;
        const uint64_t *t = a.ws.sel_ptrs + (v ? j : 0) * 6;
        const auto rg = make_rsrc(uniform_ptr(t[0]), static_cast<uint32_t>(a.I) * rowA);
        const auto rgs = make_rsrc(uniform_ptr(t[1]), static_cast<uint32_t>(a.I * GH));
        const auto ru = make_rsrc(uniform_ptr(t[2]), static_cast<uint32_t>(a.I) * rowA);
        const auto rus = make_rsrc(uniform_ptr(t[3]), static_cast<uint32_t>(a.I * GH));
#pragma unroll
        for (int u = 0; u < GA; ++u) {
            const int g = u * 64 + lane;
            const bool ok = v && g < GH;
            const uint32_t off = ok ? static_cast<uint32_t>(i) * rowA + g * 16u : kOobOffset;
            const uint32_t soff = ok ? static_cast<uint32_t>(i * GH + g) : kOobOffset;
            wg[p][u] = buf_load16_nt(rg, off);
            wu[p][u] = buf_load16_nt(ru, off);
            sg[p][u] = __builtin_amdgcn_raw_buffer_load_b8(rgs, soff, 0, 2);
            su[p][u] = __builtin_amdgcn_raw_buffer_load_b8(rus, soff, 0, 2);
        }
    }
    x_store<XT, XREG, true>(smem, xr);
    __syncthreads();
    float accg[kRoutedPairs], accu[kRoutedPairs];
#pragma unroll
    for (int p = 0; p < kRoutedPairs; ++p) accg[p] = accu[p] = 0.f;
#pragma unroll
    for (int p = 0; p < kRoutedPairs; ++p) {
#pragma unroll
        for (int u = 0; u < GA; ++u) {
            const int g = u * 64 + lane;
            if (g < GH) {
                XChunk<XT> xc[CPGX];
#pragma unroll
                for (int q = 0; q < CPGX; ++q) xc[q] = reinterpret_cast<const XChunk<XT> *>(smem)[XTile<XT>::slot(g, q)];
                accg[p] = fmaf(group_dot(wg[p][u], xc), e8m0_to_f32(sg[p][u]), accg[p]);
                accu[p] = fmaf(group_dot(wu[p][u], xc), e8m0_to_f32(su[p][u]), accu[p]);
            }
        }
    }
#pragma unroll
    for (int p = 0; p < kRoutedPairs; ++p) {
        const float g = wave_sum_to_lane63(accg[p]);
        const float u = wave_sum_to_lane63(accu[p]);
        if (lane == 63 && vv[p]) a.ws.act[static_cast<int64_t>(jj[p]) * a.I + ii[p]] = act_fn(g, u, a.act_kind, a.beta, a.lbeta);
    }
}

// ------------------------------------------------------------------ L3
// Block: 4 waves on selected expert j = blockIdx.x % k and row range rr = blockIdx.x / k of
// 4 * RW down rows (RW consecutive rows per wave).  A down row is cut into pieces of S
// elements (S = 32: one group, 16 bytes; S = 16: half a group, 8 bytes); lane l takes pieces
// l, l + 64, ... (NP of them), so each of the wave's loads is one contiguous run of the row,
// and it holds the act values of those pieces in registers for all RW rows.  The block reads
// expert j's act vector from memory once and passes it to its waves through LDS in
// chunk-major order ([chunk][piece], so the lanes of a wave read consecutive 16-byte slots)
// rather than each wave reading it again.  The row totals go to yrow[j]; the last of the range's k blocks to finish combines them in slot
// order, so the result does not depend on the order in which the blocks finish.
template <int S, int NP, int RW>
__global__ __launch_bounds__(256, 4) void layer_l3(LayerArgs a) {
    static_assert(S == 16 || S == 32, "a piece is half a group or one group");
    constexpr int ND = S / 8;   // packed dwords per piece
    constexpr int NC = S / 4;   // float4 act chunks per piece
    constexpr int RB = 4 * RW;  // rows per block
    constexpr int NA = S * NP / 16;  // act float4 per thread: the block covers I <= S * NP * 64
    __shared__ uint32_t last_s;
    __shared__ float4 act_s[NA * 256 + 1];  // expert j's act, [chunk q][piece]; the last slot is a sink
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    // slot-major order: consecutive blocks read different rows of one expert, so every XCD
    // streams from every selected expert
    const int nR = (a.Hr + RB - 1) / RB;
    const int j = blockIdx.x / nR, rr = blockIdx.x % nR;
    const int GI = a.I >> 5, P = a.I / S;
    const uint32_t rowB = static_cast<uint32_t>(a.I >> 1);
    const int n0 = rr * RB + wave * RW;
    const uint64_t *t = a.ws.sel_ptrs + j * 6;
    const auto rd = make_rsrc(uniform_ptr(t[4]), static_cast<uint32_t>(a.Hr) * rowB);
    const auto rds = make_rsrc(uniform_ptr(t[5]), static_cast<uint32_t>(a.Hr * GI));
    const auto ra = make_rsrc(a.ws.act + static_cast<int64_t>(j) * a.I, static_cast<uint32_t>(a.I) * 4u);
    // 1. expert j's act vector (one read per block; float4 c is chunk (4c % S) / 4 of piece
    //    4c / S), the wave's down rows and their scale bytes; the act goes to LDS once its
    //    loads, issued first, have arrived
    float4 ag[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int c = i * 256 + static_cast<int>(threadIdx.x);
        ag[i] = __builtin_bit_cast(float4, buf_load16(ra, c < a.I / 4 ? c * 16u : kOobOffset));
    }
    uint32_t wd[RW][NP][ND];
    uint32_t sd[RW][NP];
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
            sd[r][p] = __builtin_amdgcn_raw_buffer_load_b8(
                rds, ok ? static_cast<uint32_t>(n * GI + pc * S / 32) : kOobOffset, 0, 2);
        }
    __builtin_amdgcn_sched_barrier(0);  // every load in flight before the first wait
    // Unconditional stores and reads: chunks past I store their zeros into the sink slot, and
    // pieces past P read it (such pieces exist exactly when such chunks do) against zero
    // weights.  A store or read under a branch lets the compiler move the act load behind the
    // weight loads or wait for the weights before the first read, and then no row's dot
    // overlaps the arrival of the later rows.
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int c = i * 256 + static_cast<int>(threadIdx.x);
        act_s[c < a.I / 4 ? (c % NC) * P + c / NC : NA * 256] = ag[i];
    }
    __syncthreads();
    float4 av[NP][NC];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const int pc = p * 64 + lane;
#pragma unroll
        for (int q = 0; q < NC; ++q) av[p][q] = act_s[pc < P ? q * P + pc : NA * 256];
    }
    // 2. row dots (out-of-range pieces hold zeros); wave totals to the workspace
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int p = 0; p < NP; ++p) acc = fmaf(piece_dot<ND>(wd[r][p], av[p]), e8m0_to_f32(sd[r][p]), acc);
        const float tot = wave_sum_to_lane63(acc);
        const int n = n0 + r;
        if (lane == 63 && n < a.Hr)
            __hip_atomic_store(a.ws.yrow + static_cast<int64_t>(j) * a.Hr + n, tot, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    // 3. the block counts itself done once its row stores (agent-scope atomic stores) have
    //    completed; the last of the range's k blocks runs an agent-scope acquire, resets the
    //    counter and combines.  L2 zeroed every range counter before this launch, so stale
    //    counter bytes cannot skip or misplace the combine.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t *c = a.ws.counter + 1 + rr;
        const uint32_t old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_s = old + 1 == static_cast<uint32_t>(a.k);
        if (last_s) {
            __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
    }
    __syncthreads();
    if (!last_s) return;
    const int n = rr * RB + static_cast<int>(threadIdx.x);
    if (static_cast<int>(threadIdx.x) >= RB || n >= a.Hr) return;
    // 4. y = sum_j w_j * down_j in slot order (latent layer: the routed sum in latent space,
    //    for the norm and up projection of L4), plus the shared expert's row.  The row totals
    //    are read with device-coherent loads, all issued before the sum (slot indices past k
    //    are clamped and their terms dropped).
    const auto rw = make_rsrc(a.ws.topk_w, static_cast<uint32_t>(a.k) * 4u);
    float v[kMaxTopK], tw[kMaxTopK];
#pragma unroll
    for (int jj = 0; jj < kMaxTopK; ++jj) {
        const int js = jj < a.k ? jj : a.k - 1;
        v[jj] = __hip_atomic_load(a.ws.yrow + static_cast<int64_t>(js) * a.Hr + n, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
        tw[jj] = __builtin_bit_cast(float, buf_load4(rw, jj * 4u));
    }
    float y = 0.f;
#pragma unroll
    for (int jj = 0; jj < kMaxTopK; ++jj) y = jj < a.k ? fmaf(tw[jj], v[jj], y) : y;
    if (a.lat_down) {
        a.ws.ylat[n] = y;
        return;
    }
    if (a.sh_down) y += a.ws.yshared[n];
    if (a.out_bf16)
        static_cast<uint16_t *>(a.out)[n] = f32_to_bf16(y);
    else
        static_cast<float *>(a.out)[n] = y;
}


// The router arrival counter back to zero (the route-only call, which has no L2 to do it).
__global__ void counter_zero_kernel(uint32_t *counter) {
    if (threadIdx.x == 0) counter[0] = 0u;
}

// ------------------------------------------------------------------ host side
struct LayerWsLayout {
    size_t logits, scores, corrected, idx, w, shared_act, act, yshared, ptrs, counter, h, ylat, yrow, total;
};

static size_t up256(size_t v) { return (v + 255) & ~size_t(255); }

// The arrival counters sit in the first kCounterBytes for every shape, so workspaces shared
// by layers of different shapes keep them at one place (zero between calls); the records
// after them are rewritten by every call.
static LayerWsLayout layer_ws_layout(int64_t H, int64_t I, int64_t Is, int64_t E, int64_t k, int64_t Hr = 0) {
    LayerWsLayout L{};
    size_t o = 0;
    L.counter = o, o += kCounterBytes;
    L.logits = o, o += up256(E * 4);
    L.scores = o, o += up256(E * 4);
    L.corrected = o, o += up256(E * 4);
    L.idx = o, o += up256(k * 4);
    L.w = o, o += up256(k * 4);
    L.shared_act = o, o += up256(std::max<int64_t>(Is, 1) * 4);
    L.act = o, o += up256(k * I * 4);
    L.yshared = o, o += up256(H * 4);
    L.ptrs = o, o += up256(k * 6 * 8);
    L.h = o, o += up256(Hr * 4);
    L.ylat = o, o += up256(Hr * 4);
    L.yrow = o, o += up256(k * std::max(H, Hr) * 4);
    L.total = o;
    return L;
}

// Whether a grid of `blocks` blocks of layer_l1<XT, C> is resident all at once on the current
// device (CUs x blocks per CU at the kernel's occupancy), computed once per device.
constexpr int kMaxDevices = 64;
template <typename XT, int C, bool D>
static bool l1_one_round(int blocks, size_t lds) {
    // blocks held at once + 1; 0: not computed yet (threads that race here store one value)
    static std::atomic<int> resident[kMaxDevices] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
    int r = resident[dev].load(std::memory_order_relaxed);
    if (!r) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, layer_l1<XT, C, D>, 256, lds) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return false;
        r = per_cu * cus + 1;
        resident[dev].store(r, std::memory_order_relaxed);
    }
    return blocks < r;
}

template <typename XT>
static int launch_l1(LayerArgs &a, bool with_shared, hipStream_t st) {
    const int chh = static_cast<int>(cdiv(a.H / 8, 64));
    a.l1_router_blocks = static_cast<int>(cdiv(a.E, 4));
    a.l1_latent_blocks = a.lat_down ? static_cast<int>(cdiv(a.Hr, 4)) : 0;
    const int blocks = a.l1_router_blocks + a.l1_latent_blocks + (with_shared ? static_cast<int>(cdiv(a.Is, 4)) : 0);
    const size_t lds = static_cast<size_t>(256) * x_regs<XT>() * 16;
#define K3_L1(C) \
    if (chh <= C) { \
        if (!a.lat_down && with_shared && l1_one_round<XT, C, true>(blocks, lds)) \
            layer_l1<XT, C, true><<<dim3(blocks), 256, lds, st>>>(a); \
        else \
            layer_l1<XT, C, false><<<dim3(blocks), 256, lds, st>>>(a); \
        return check_hip(hipGetLastError(), "moe layer L1"); \
    }
    K3_L1(4) K3_L1(8) K3_L1(12) K3_L1(16)
#undef K3_L1
    return set_error(K3_ERR_SHAPE, "moe layer: H=%d too wide", a.H);
}

// L4 of the latent layer (nothing to do for the plain layer): the dense rows of W_up against
// rmsnorm(ylat) * norm (every block normalises the latent sum itself), plus the shared row
static int launch_l4(const LayerArgs &a, hipStream_t st) {
    if (!a.lat_down) return K3_OK;
    RowsArgs r{};
    r.src = a.ws.ylat, r.nw = a.lat_norm, r.eps = a.eps, r.K = a.Hr;
    r.w[0] = a.lat_up, r.N[0] = a.H;
    r.out = a.out, r.out_bf16 = a.out_bf16, r.add = a.sh_down ? a.ws.yshared : nullptr;
    return launch_rows<kModeNorm>(r, st);
}

template <typename XT>
static int launch_layer(LayerArgs &a, hipStream_t st) {
    const int GH = a.Hr / 32, GI = a.I / 32;
    const int chi = static_cast<int>(cdiv(a.Is / 8, 64));
    const int ga = GH <= 64 ? 1 : (GH <= 128 ? 2 : (GH <= 256 ? 4 : 0));
    const int gb = GI <= 64 ? 1 : (GI <= 128 ? 2 : 0);
    if (!ga || !gb || (a.sh_down && chi > 16))
        return set_error(K3_ERR_SHAPE, "moe layer: H=%d I=%d Is=%d outside the kernels' range", a.H, a.I, a.Is);
    const int rb = GI <= 64 ? 4 * 14 : (GI <= 96 ? 4 * 7 : 4 * 4);  // L3 rows per block
    a.l3_ranges = static_cast<int>(cdiv(a.Hr, rb));
    if (1 + a.l3_ranges > static_cast<int>(kCounterBytes / 4))
        return set_error(K3_ERR_SHAPE, "moe layer: %d rows need more row-range counters than the workspace holds",
                         a.Hr);
    int rc = launch_l1<XT>(a, a.sh_gate != nullptr, st);
    if (rc) return rc;
    // L2 (zeroes the arrival counters L3 uses)
    const int chi_l2 = chi <= 4 ? 4 : (chi <= 8 ? 8 : 16);
    a.l2_shared_blocks = a.sh_down ? static_cast<int>(cdiv(a.H, 4 * shared_down_rows(chi_l2))) : 0;
    const int routed_blocks = static_cast<int>(cdiv(static_cast<int64_t>(a.k) * a.I, 4 * kRoutedPairs));
    const size_t lds2 = static_cast<size_t>(256) * x_regs<XT>() * 16;
    const dim3 g2(static_cast<unsigned>(a.l2_shared_blocks + routed_blocks));
#define K3_L2(G_, C_) \
    if (ga == G_ && (chi <= C_ || !a.sh_down)) { \
        layer_l2<XT, G_, C_><<<g2, 256, lds2, st>>>(a); \
    } else
    K3_L2(1, 4) K3_L2(1, 8) K3_L2(1, 16) K3_L2(2, 4) K3_L2(2, 8) K3_L2(2, 16) K3_L2(4, 4) K3_L2(4, 8)
    K3_L2(4, 16) {
        return set_error(K3_ERR_SHAPE, "moe layer: no L2 kernel for H=%d Is=%d", a.H, a.Is);
    }
#undef K3_L2
    rc = check_hip(hipGetLastError(), "moe layer L2");
    if (rc) return rc;
    // L3: pieces of a down row per lane and rows per wave, so a lane's act values and its
    // rows' weights fit in about 128 registers (four blocks per CU)
    const dim3 g3(static_cast<unsigned>(a.k * a.l3_ranges));
    if (GI <= 64)
        layer_l3<32, 1, 14><<<g3, 256, 0, st>>>(a);
    else if (GI <= 96)
        layer_l3<16, 3, 7><<<g3, 256, 0, st>>>(a);
    else
        layer_l3<32, 2, 4><<<g3, 256, 0, st>>>(a);
    rc = check_hip(hipGetLastError(), "moe layer L3");
    return rc ? rc : launch_l4(a, st);
}

}  // namespace k3

using namespace k3;

extern "C" int64_t k3_moe_layer_workspace_size(int64_t H, int64_t I, int64_t shared_I, int64_t n_experts,
                                               int64_t top_k) {
    return static_cast<int64_t>(layer_ws_layout(H, I, shared_I, n_experts, top_k).total);
}

static int layer_impl(const void *x, int x_dtype, const void *router_w, const void *router_bias, int route_kind,
                      int renormalize, float scaling, const void *expert_table, const void *shared_gate,
                      const void *shared_up, const void *shared_down, void *out, int out_dtype, int64_t H, int64_t I,
                      int64_t shared_I, int64_t n_experts, int64_t top_k, int act_kind, float beta, float linear_beta,
                      void *workspace, int64_t workspace_bytes, void *stream, bool route_only_flag,
                      const void *lat_down = nullptr, const void *lat_up = nullptr, const void *lat_norm = nullptr,
                      float eps = 0.f, int64_t latent = 0) {
    if (!x || !router_w || !workspace || (!route_only_flag && (!expert_table || !out)))
        return set_error(K3_ERR_NULL, "moe layer: null pointer");
    const bool lat = lat_down != nullptr;
    if (lat) {
        if (!lat_up || !lat_norm) return set_error(K3_ERR_NULL, "moe latent layer: null pointer");
        if (latent <= 0 || latent % 128 || latent > 8192)
            return set_error(K3_ERR_SHAPE, "moe latent layer: latent=%lld must be a positive multiple of 128, <= 8192",
                             (long long)latent);
        if (!aligned16(lat_down) || !aligned16(lat_up) || !aligned16(lat_norm))
            return set_error(K3_ERR_ALIGN, "moe latent layer: projections must be 16-byte aligned");
        if (latent * H * 2 >= (1ll << 31) || latent * I / 2 >= (1ll << 31))
            return set_error(K3_ERR_SHAPE, "moe latent layer: a weight matrix exceeds 2 GiB");
    }
    const bool has_shared = shared_gate || shared_up || shared_down;
    if (has_shared && !(shared_gate && shared_up && shared_down))
        return set_error(K3_ERR_NULL, "moe layer: shared expert needs gate, up and down");
    if (x_dtype != K3_F32 && x_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "moe layer: x_dtype");
    if (out_dtype != K3_F32 && out_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "moe layer: out_dtype");
    if (route_kind != K3_ROUTE_SOFTMAX && route_kind != K3_ROUTE_SIGMOID_BIAS)
        return set_error(K3_ERR_SHAPE, "moe layer: route_kind");
    if (act_kind != K3_ACT_SILU && act_kind != K3_ACT_SITU) return set_error(K3_ERR_SHAPE, "moe layer: act_kind");
    if (H <= 0 || I <= 0 || H % 128 || I % 128 || H > 8192 || (has_shared && (shared_I <= 0 || shared_I % 128)))
        return set_error(K3_ERR_SHAPE,
                         "moe layer: H, I and shared_I must be positive multiples of 128, H <= 8192");
    if (n_experts <= 0 || n_experts > kMaxExperts || top_k <= 0 || top_k > kMaxTopK || top_k > n_experts)
        return set_error(K3_ERR_SHAPE, "moe layer: n_experts must be in 1..%d and top_k in 1..min(%d, n_experts)",
                         kMaxExperts, kMaxTopK);
    const LayerWsLayout L = layer_ws_layout(H, I, has_shared ? shared_I : 0, n_experts, top_k, lat ? latent : 0);
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
    a.ws.counter = reinterpret_cast<uint32_t *>(w + L.counter);
    a.ws.yrow = reinterpret_cast<float *>(w + L.yrow);
    a.H = static_cast<int>(H);
    a.Hr = static_cast<int>(lat ? latent : H);
    if (lat) {
        a.lat_down = static_cast<const uint16_t *>(lat_down);
        a.lat_up = static_cast<const uint16_t *>(lat_up);
        a.lat_norm = static_cast<const float *>(lat_norm);
        a.eps = eps;
        a.ws.h = w + L.h;
        a.ws.ylat = reinterpret_cast<float *>(w + L.ylat);
    }
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
    if (route_only_flag) {
        // Only L1 runs, and no later launch of this call zeroes the router counter: zero it
        // first, so a workspace whose counter bytes hold garbage still routes on this call.
        counter_zero_kernel<<<1, 64, 0, st>>>(a.ws.counter);
        const int rc = check_hip(hipGetLastError(), "moe route: counter reset");
        if (rc) return rc;
        return x_dtype == K3_BF16 ? launch_l1<uint16_t>(a, false, st) : launch_l1<float>(a, false, st);
    }
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

extern "C" int64_t k3_moe_latent_layer_workspace_size(int64_t H, int64_t latent, int64_t I, int64_t shared_I,
                                                      int64_t n_experts, int64_t top_k) {
    return static_cast<int64_t>(layer_ws_layout(H, I, shared_I, n_experts, top_k, latent).total);
}

extern "C" int k3_moe_latent_layer_decode(const void *x, int x_dtype, const void *router_w, const void *router_bias,
                                          int renormalize, float scaling, const void *expert_table,
                                          const void *latent_down, const void *latent_up, const void *latent_norm,
                                          float eps, const void *shared_gate, const void *shared_up,
                                          const void *shared_down, void *out, int out_dtype, int64_t H,
                                          int64_t latent, int64_t I, int64_t shared_I, int64_t n_experts,
                                          int64_t top_k, int act_kind, float beta, float linear_beta,
                                          void *workspace, int64_t workspace_bytes, void *stream) {
    if (!latent_down) return set_error(K3_ERR_NULL, "moe latent layer: null pointer");
    return layer_impl(x, x_dtype, router_w, router_bias, K3_ROUTE_SIGMOID_BIAS, renormalize, scaling, expert_table,
                      shared_gate, shared_up, shared_down, out, out_dtype, H, I, shared_I, n_experts, top_k, act_kind,
                      beta, linear_beta, workspace, workspace_bytes, stream, false, latent_down, latent_up,
                      latent_norm, eps, latent);
}

extern "C" int k3_moe_route(const void *x, int x_dtype, const void *router_w, const void *router_bias, int route_kind,
                            int renormalize, float scaling, int64_t H, int64_t n_experts, int64_t top_k,
                            void *workspace, int64_t workspace_bytes, void *stream) {
    return layer_impl(x, x_dtype, router_w, router_bias, route_kind, renormalize, scaling, nullptr, nullptr, nullptr,
                      nullptr, nullptr, K3_F32, H, 128, 0, n_experts, top_k, K3_ACT_SILU, 1.f, 0.f, workspace,
                      workspace_bytes, stream, true);
}

extern "C" int k3_moe_topk(const float *logits, int64_t ld_logits, int64_t T, int64_t n_experts,
                           const float *router_bias, int route_kind, int renormalize, float scaling, int64_t top_k,
                           int32_t *expert_idx, float *expert_w, float *scores, float *corrected, void *stream) {
    if (T < 0) return set_error(K3_ERR_SHAPE, "moe topk: T=%lld", (long long)T);
    if (route_kind != K3_ROUTE_SOFTMAX && route_kind != K3_ROUTE_SIGMOID_BIAS)
        return set_error(K3_ERR_SHAPE, "moe topk: route_kind");
    if (n_experts <= 0 || n_experts > kMaxExperts || top_k <= 0 || top_k > kMaxTopK || top_k > n_experts)
        return set_error(K3_ERR_SHAPE, "moe topk: n_experts must be in 1..%d and top_k in 1..min(%d, n_experts)",
                         kMaxExperts, kMaxTopK);
    if (ld_logits < n_experts) return set_error(K3_ERR_SHAPE, "moe topk: ld_logits < n_experts");
    if (T == 0) return K3_OK;
    if (!logits || !expert_idx || !expert_w || !scores || !corrected)
        return set_error(K3_ERR_NULL, "moe topk: null pointer");
    if (T > (1ll << 31) - 1) return set_error(K3_ERR_SHAPE, "moe topk: T too large");
    LayerArgs a{};
    a.router_bias = router_bias;
    a.E = static_cast<int>(n_experts);
    a.k = static_cast<int>(top_k);
    a.route_kind = route_kind;
    a.renorm = renormalize;
    a.scaling = scaling;
    a.ws.logits = const_cast<float *>(logits);
    a.ws.scores = scores;
    a.ws.corrected = corrected;
    a.ws.topk_idx = expert_idx;
    a.ws.topk_w = expert_w;
    topk_kernel<<<dim3(static_cast<unsigned>(T)), 256, 0, static_cast<hipStream_t>(stream)>>>(a, ld_logits);
    return check_hip(hipGetLastError(), "moe topk launch");
}

extern "C" int k3_moe_layer_workspace_offsets(int64_t H, int64_t I, int64_t shared_I, int64_t n_experts,
                                              int64_t top_k, int64_t *offsets) {
    if (!offsets) return set_error(K3_ERR_NULL, "moe layer offsets: null pointer");
    const LayerWsLayout L = layer_ws_layout(H, I, shared_I, n_experts, top_k);
    const size_t v[8] = {L.logits, L.scores, L.corrected, L.idx, L.w, L.shared_act, L.act, L.yshared};
    for (int i = 0; i < 8; ++i) offsets[i] = static_cast<int64_t>(v[i]);
    return K3_OK;
}
