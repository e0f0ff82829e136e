// Dense bf16 row kernels for batch-1 decode steps: a launch takes up to six row sets
// [N, K] (bf16, row-major) that share one fp32 input vector of K values, staged in LDS,
// and writes one fp32 dot product per row.  The vector is built in the prologue:
//   kModeX         x itself (bf16 or fp32)
//   kModeNorm      rmsnorm(src) * nw over all K values (every block normalises it)
//   kModeGate      a fp32 vector as is (gl null) or times sigmoid(gl)
//   kModeHeadNorm  per head of 128 values: o * nw[i] / rms(head), the head's sum of squares
//                  given as four partial sums in gl (o already carries its gate)
// Every block issues its weight rows first, then stages the vector, then reduces: a lane
// takes 16-byte chunks (8 bf16) l, l + 64, ... of a row; R rows per wave, 4 waves (8 for
// rows of more than 2048 values, so one staged vector serves more rows).
#pragma once

#include <algorithm>
#include <atomic>

#include "k3_common.h"

namespace k3 {
namespace {

enum { kModeX = 0, kModeNorm = 1, kModeGate = 2, kModeHeadNorm = 3 };
constexpr int kRowSets = 6;
constexpr int kMaxWidth = 12288;  // input vector width (fp32 in LDS: 48 KB)

struct RowsArgs {
    const void *x;            // kModeX: [K] bf16 or fp32
    int x_bf16;
    const float *src, *nw;    // kModeNorm: v = src * rsqrt(mean(src^2) + eps) * nw
    float eps;
    const float *o, *gl;      // kModeGate / kModeHeadNorm: the vector and its gate logits
    int K;
    const uint16_t *w[kRowSets];   // bf16 row sets [N, K] sharing v (null: unused)
    int N[kRowSets];
    int blocks[kRowSets];
    float *y[kRowSets];            // fp32 outputs [N] (when out is null)
    void *out;                     // not null: set 0's outputs go here, fp32 or bf16
    int out_bf16;
    const float *add;              // with out: added to each output row (null: nothing)
    // kModeNorm, last block: the cache append
    const float *ckv, *kvw;   // ckv [r + rope] fp32, kv_a_layernorm [r]
    uint16_t *lat_row, *rot_row;
    int r, rope, append;
};

template <int NW>
__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum_all(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) t += red[w];
    __syncthreads();
    return t;
}

// v (fp32, K values) into LDS; ends with a block barrier.  CH bounds K (K <= 512 CH), so a
// thread's share is at most NF float4 chunks (c = j * NT + threadIdx.x); they are loaded in
// batches of VB chunks with every load of a batch issued before any is used (buffer loads:
// past the end, zeros and no access), so the staging costs one memory round trip per batch.
template <int MODE, int NW, int CH>
__device__ __forceinline__ void stage_vector(const RowsArgs &a, float *vs, float *red) {
    constexpr int NT = 64 * NW;
    constexpr int NF = (2 * CH + NW - 1) / NW;  // float4 chunks per thread
    constexpr int VB = CH >= 24 ? 2 : 4;         // chunks per batch (registers beside the rows)
    const int K = a.K, n4 = K / 4;
    const int tid = static_cast<int>(threadIdx.x);
    float4 *v4 = reinterpret_cast<float4 *>(vs);
    auto off = [tid](int j) { return static_cast<uint32_t>(j * NT + tid) * 16u; };
    if (MODE == kModeX) {
        if (a.x_bf16) {
            constexpr int NB = (CH + NW - 1) / NW;  // 16-byte bf16 chunks per thread
            const auto rx = make_rsrc(a.x, static_cast<uint32_t>(K) * 2u);
            uint4 q[NB];
#pragma unroll
            for (int j = 0; j < NB; ++j) q[j] = buf_load16(rx, off(j));
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int c = j * NT + tid;
                if (c < K / 8) {
                    const uint32_t d[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        vs[8 * c + 2 * i] = __uint_as_float(d[i] << 16);
                        vs[8 * c + 2 * i + 1] = __uint_as_float(d[i] & 0xffff0000u);
                    }
                }
            }
        } else {
            const auto rx = make_rsrc(a.x, static_cast<uint32_t>(K) * 4u);
#pragma unroll
            for (int j0 = 0; j0 < NF; j0 += VB) {
                float4 q[VB];
#pragma unroll
                for (int j = 0; j < VB; ++j) q[j] = __builtin_bit_cast(float4, buf_load16(rx, off(j0 + j)));
#pragma unroll
                for (int j = 0; j < VB; ++j)
                    if ((j0 + j) * NT + tid < n4) v4[(j0 + j) * NT + tid] = q[j];
            }
        }
    } else if (MODE == kModeNorm) {
        // src and nw of the batch together; the sum of squares in the lane's chunk order
        const auto rsrc = make_rsrc(a.src, static_cast<uint32_t>(K) * 4u);
        const auto rnw = make_rsrc(a.nw, static_cast<uint32_t>(K) * 4u);
        float4 sv[NF], gv[NF];
        float ss = 0.f;
#pragma unroll
        for (int j0 = 0; j0 < NF; j0 += VB) {
#pragma unroll
            for (int j = j0; j < j0 + VB && j < NF; ++j) {
                sv[j] = __builtin_bit_cast(float4, buf_load16(rsrc, off(j)));
                gv[j] = __builtin_bit_cast(float4, buf_load16(rnw, off(j)));
            }
#pragma unroll
            for (int j = j0; j < j0 + VB && j < NF; ++j) {
                const float4 x = sv[j];
                ss = fmaf(x.x, x.x, fmaf(x.y, x.y, fmaf(x.z, x.z, fmaf(x.w, x.w, ss))));
            }
        }
        const float rs = 1.0f / sqrtf(block_sum<NW>(ss, red) / static_cast<float>(K) + a.eps);
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const int c = j * NT + tid;
            if (c < n4) {
                float4 v = sv[j];
                const float4 g = gv[j];
                v.x = v.x * rs * g.x, v.y = v.y * rs * g.y, v.z = v.z * rs * g.z, v.w = v.w * rs * g.w;
                v4[c] = v;
            }
        }
    } else if (MODE == kModeHeadNorm) {
        // heads of 128 values = 32 float4; gl holds four partial sums of squares per head
        const auto ro = make_rsrc(a.o, static_cast<uint32_t>(K) * 4u);
        const auto rgl = make_rsrc(a.gl, static_cast<uint32_t>(K / 128) * 16u);
        const auto rnw = make_rsrc(a.nw, 128u * 4u);
#pragma unroll
        for (int j0 = 0; j0 < NF; j0 += VB) {
            float4 ov[VB], pv[VB], wv[VB];
#pragma unroll
            for (int j = 0; j < VB; ++j) {
                const int c = (j0 + j) * NT + tid;
                ov[j] = __builtin_bit_cast(float4, buf_load16(ro, off(j0 + j)));
                pv[j] = __builtin_bit_cast(float4, buf_load16(rgl, c < n4 ? static_cast<uint32_t>(c >> 5) * 16u : kOobOffset));
                wv[j] = __builtin_bit_cast(float4, buf_load16(rnw, static_cast<uint32_t>(c & 31) * 16u));
            }
#pragma unroll
            for (int j = 0; j < VB; ++j) {
                const int c = (j0 + j) * NT + tid;
                if (c < n4) {
                    const float4 p = pv[j], w = wv[j];
                    const float rs = 1.0f / sqrtf((((p.x + p.y) + p.z) + p.w) / 128.0f + a.eps);
                    float4 v = ov[j];
                    v.x = v.x * rs * w.x, v.y = v.y * rs * w.y, v.z = v.z * rs * w.z, v.w = v.w * rs * w.w;
                    v4[c] = v;
                }
            }
        }
    } else {
        const auto ro = make_rsrc(a.o, static_cast<uint32_t>(K) * 4u);
        const auto rgl = make_rsrc(a.gl, a.gl ? static_cast<uint32_t>(K) * 4u : 0u);
#pragma unroll
        for (int j0 = 0; j0 < NF; j0 += VB) {
            float4 ov[VB], gv[VB];
#pragma unroll
            for (int j = 0; j < VB; ++j) {
                ov[j] = __builtin_bit_cast(float4, buf_load16(ro, off(j0 + j)));
                gv[j] = __builtin_bit_cast(float4, buf_load16(rgl, off(j0 + j)));
            }
#pragma unroll
            for (int j = 0; j < VB; ++j) {
                const int c = (j0 + j) * NT + tid;
                if (c < n4) {
                    float4 v = ov[j];
                    if (a.gl) {
                        const float4 g = gv[j];
                        v.x /= 1.0f + expf(-g.x), v.y /= 1.0f + expf(-g.y), v.z /= 1.0f + expf(-g.z),
                            v.w /= 1.0f + expf(-g.w);
                    }
                    v4[c] = v;
                }
            }
        }
    }
    __syncthreads();
}

// c_new = rmsnorm(ckv[:r]) * kv_a_layernorm -> lat_row (bf16); rot_row = bf16(ckv[r:])
template <int NW>
__device__ void append_row(const RowsArgs &a, float *red) {
    constexpr int NT = 64 * NW;
    float ss = 0.f;
    for (int j = threadIdx.x; j < a.r; j += NT) ss = fmaf(a.ckv[j], a.ckv[j], ss);
    const float rs = 1.0f / sqrtf(block_sum<NW>(ss, red) / static_cast<float>(a.r) + a.eps);
    for (int j = threadIdx.x; j < a.r; j += NT) a.lat_row[j] = f32_to_bf16(a.ckv[j] * rs * a.kvw[j]);
    for (int j = threadIdx.x; j < a.rope; j += NT) a.rot_row[j] = f32_to_bf16(a.ckv[a.r + j]);
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

// Block: NW waves x R rows of one row set; CH 16-byte chunks per lane per row.
template <int MODE, int CH, int R, int NW>
__global__ __launch_bounds__(64 * NW) void step_rows_kernel(RowsArgs a) {
    extern __shared__ float vs[];
    __shared__ float red[NW];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (MODE == kModeNorm && a.append && static_cast<int>(blockIdx.x) == static_cast<int>(gridDim.x) - 1) {
        append_row<NW>(a, red);
        return;
    }
    int b = blockIdx.x, s = 0;
    while (s < kRowSets - 1 && b >= a.blocks[s]) b -= a.blocks[s++];
    const int N = a.N[s], K = a.K, nch = K >> 3;
    const uint32_t rowb = static_cast<uint32_t>(K) * 2u;
    const int n0 = (b * NW + wave) * R;
    const auto rw = make_rsrc(a.w[s], static_cast<uint32_t>(N) * rowb);
    // 1. the wave's rows
    uint4 wr[R][CH];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int c = u * 64 + lane, n = n0 + r;
            wr[r][u] = buf_load16_nt(rw, (n < N && c < nch) ? static_cast<uint32_t>(n) * rowb + c * 16u : kOobOffset);
        }
    // 2. the input vector
    stage_vector<MODE, NW, CH>(a, vs, red);
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
            if (a.out) {
                const float t2 = a.add ? t + a.add[n] : t;
                if (a.out_bf16)
                    static_cast<uint16_t *>(a.out)[n] = f32_to_bf16(t2);
                else
                    static_cast<float *>(a.out)[n] = t2;
            } else {
                a.y[s][n] = t;
            }
        }
    }
}

// Persistent form for wide rows: about one block per CU walks the row groups
// g = blockIdx.x, blockIdx.x + gridDim.x, ... of the concatenated row sets (NW rows per group,
// one per wave, a.blocks[s] groups in set s).  The input vector is staged once per block and
// every wave keeps the next group's row in flight while it reduces the current one, so no
// block restages the vector and the CUs share the rows evenly.  No cache append.
template <int MODE, int CH, int NW>
__global__ __launch_bounds__(64 * NW) void step_rows_loop_kernel(RowsArgs a) {
    extern __shared__ float vs[];
    __shared__ float red[NW];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int K = a.K, nch = K >> 3;
    const uint32_t rowb = static_cast<uint32_t>(K) * 2u;
    int total = 0;
#pragma unroll
    for (int s = 0; s < kRowSets; ++s) total += a.blocks[s];
    const int G = static_cast<int>(gridDim.x);
    // this wave's row of group g: set s, row n (none when g >= total or n >= N[s]; such rows
    // load zeros through out-of-range offsets and store nothing)
    auto locate = [&](int g, int &s, int &n) {
        int b = g;
        s = 0;
        while (s < kRowSets - 1 && b >= a.blocks[s]) b -= a.blocks[s++];
        n = b * NW + wave;
    };
    auto load_row = [&](uint4 (&wr)[CH], int g) {
        int s, n;
        locate(g, s, n);
        const bool ok = g < total && n < a.N[s];
        const auto rw = make_rsrc(a.w[s], static_cast<uint32_t>(a.N[s]) * rowb);
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int c = u * 64 + lane;
            wr[u] = buf_load16_nt(rw, (ok && c < nch) ? static_cast<uint32_t>(n) * rowb + c * 16u : kOobOffset);
        }
    };
    auto reduce_row = [&](const uint4 (&wr)[CH], int g) {
        int s, n;
        locate(g, s, n);
        const float4 *v4 = reinterpret_cast<const float4 *>(vs);
        float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int c = u * 64 + lane;
            if (c < nch) {
                if (u & 1)
                    acc1 = dot8_bf16_f32(wr[u], v4[2 * c], v4[2 * c + 1], acc1);
                else
                    acc0 = dot8_bf16_f32(wr[u], v4[2 * c], v4[2 * c + 1], acc0);
            }
        }
        const float t = wave_sum_to_lane63(acc0 + acc1);
        if (lane == 63 && g < total && n < a.N[s]) {
            if (a.out) {
                const float t2 = a.add ? t + a.add[n] : t;
                if (a.out_bf16)
                    static_cast<uint16_t *>(a.out)[n] = f32_to_bf16(t2);
                else
                    static_cast<float *>(a.out)[n] = t2;
            } else {
                a.y[s][n] = t;
            }
        }
    };
    uint4 wa[CH], wb[CH];
    int g = static_cast<int>(blockIdx.x);
    load_row(wa, g);
    stage_vector<MODE, NW, CH>(a, vs, red);
    for (; g < total; g += 2 * G) {
        load_row(wb, g + G);
        reduce_row(wa, g);
        if (g + G >= total) break;
        load_row(wa, g + 2 * G);
        reduce_row(wb, g + G);
    }
}

// Resident blocks of the persistent form per device (occupancy x CUs), cached.
template <int MODE, int CH, int NW>
int rows_loop_blocks(size_t lds) {
    constexpr int kDevs = 64;
    static std::atomic<int> cached[kDevs] = {};  // 0: not computed yet (racing threads store one value)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDevs) return 0;
    int r = cached[dev].load(std::memory_order_relaxed);
    if (!r) {
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, step_rows_loop_kernel<MODE, CH, NW>, 64 * NW, lds) !=
                hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        r = std::max(1, per_cu) * cus;
        cached[dev].store(r, std::memory_order_relaxed);
    }
    return r;
}

template <int MODE, int CH>
int launch_rows_ch(RowsArgs &a, hipStream_t st) {
    // rows of 2049..4096 values: eight waves of two rows (16 rows per staged vector);
    // rows of 4097..8192 values: eight waves of one row, so one staged vector serves 8 rows;
    // rows of 8193..12288 values: eight waves of two rows (16 rows per staged 48 KB vector).
    // Measured faster than four-wave blocks for all three.  Rows of 1025..2048 values take
    // two rows per wave in four-wave blocks (measured faster than four rows per wave).
    constexpr int R = CH >= 24 ? 2 : (CH >= 16 ? 1 : (CH >= 8 ? 2 : (CH >= 4 ? 2 : 8)));
    constexpr int NW = CH >= 8 ? 8 : 4;
    int total = 0;
    for (int s = 0; s < kRowSets; ++s) {
        a.blocks[s] = a.w[s] ? static_cast<int>(cdiv(a.N[s], NW * R)) : 0;
        total += a.blocks[s];
    }
    if (MODE == kModeNorm && a.append) ++total;
    if (total == 0) return K3_OK;  // no rows and no cache append: nothing to launch
    step_rows_kernel<MODE, CH, R, NW><<<dim3(static_cast<unsigned>(total)), 64 * NW, static_cast<size_t>(a.K) * 4, st>>>(a);
    return check_hip(hipGetLastError(), "dense rows launch");
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
    return set_error(K3_ERR_SHAPE, "dense rows: input width %d above %d", a.K, kMaxWidth);
}

// Row sets of 4097..12288 values through the persistent form (eight waves, one row each);
// other widths, and the normalising launch with the cache append, take launch_rows.
template <int MODE>
int launch_rows_loop(RowsArgs &a, hipStream_t st) {
    const int ch = static_cast<int>(cdiv(a.K / 8, 64));
    if (ch <= 8 || ch > 24 || (MODE == kModeNorm && a.append)) return launch_rows<MODE>(a, st);
    constexpr int NW = 8;
    int total = 0;
    for (int s = 0; s < kRowSets; ++s) {
        a.blocks[s] = a.w[s] ? static_cast<int>(cdiv(a.N[s], NW)) : 0;
        total += a.blocks[s];
    }
    if (total == 0) return K3_OK;
    const size_t lds = static_cast<size_t>(a.K) * 4;
    auto go = [&](auto kern, int resident) {
        if (resident <= 0) return set_error(K3_ERR_HIP, "dense rows (persistent): occupancy query failed");
        const int grid = std::max(1, std::min(total, resident));
        kern<<<dim3(static_cast<unsigned>(grid)), 64 * NW, lds, st>>>(a);
        return check_hip(hipGetLastError(), "dense rows (persistent) launch");
    };
    if (ch <= 16) return go(step_rows_loop_kernel<MODE, 16, NW>, rows_loop_blocks<MODE, 16, NW>(lds));
    return go(step_rows_loop_kernel<MODE, 24, NW>, rows_loop_blocks<MODE, 24, NW>(lds));
}

}  // namespace
}  // namespace k3
