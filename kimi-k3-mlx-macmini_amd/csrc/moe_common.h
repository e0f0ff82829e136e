// Pieces shared by the expert-FFN and MoE-layer kernels: activations and the grid-wide
// dataflow barrier of the single-launch persistent kernels.
//
// Barrier design (measured on MI355X: ~3 us per barrier at 512 blocks, against 10-180 us
// for counter-based variants with release fences or one contended atomic):
//   * one flag word per block, no read-modify-write anywhere on the arrival path;
//   * two levels: blocks 0..7 lead the groups {g, g+8, g+16, ...}; a leader polls its
//     members' flags and publishes a group flag, every block polls the 8 group flags.
//     (Measured from the last arrival to release: ~1.7-2.1 us at 256-1024 blocks, where
//     every block polling every flag takes 3-7 us from hot-spotting one memory channel);
//   * flags carry an epoch: every block reads the workspace epoch word at kernel start and
//     publishes epoch + j + 1 at barrier j; block 0 advances the epoch once barrier 0 has
//     passed, so the workspace needs no reset between launches (zero-filled once);
//   * data crossing the barrier is written and read with agent-coherent (sc1) accesses,
//     and the publishing wave waits for its stores to complete before storing its flag.
//     Only wave 0 of a block publishes: it holds no outstanding loads at that point, so
//     its wait does not serialise behind the weight prefetches of the other waves;
//   * the wait is a bounded poll: after kSpinLimit rounds it sets the workspace error
//     word and falls through (wrong results, never a hang).  Grids are sized to be fully
//     resident, which the barrier requires.
#pragma once

#include "k3_common.h"

namespace k3 {

constexpr int kMaxGridBlocks = 2048;
constexpr size_t kFlagsOffset = 256;                                  // bytes
constexpr size_t kGroupFlagsOffset = kFlagsOffset + 4 * kMaxGridBlocks; // 8448
constexpr int kGroups = 8;
constexpr int kGroupStride = 32;                                       // words: one line each
constexpr size_t kBarrierBytes = kGroupFlagsOffset + 4 * kGroups * kGroupStride;
constexpr size_t kBarrierRegion = (kBarrierBytes + 255) & ~size_t(255);
constexpr int kErrWord = 2;  // word 0: epoch, word 2: error flag
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr uint32_t kErrBarrierTimeout = 1u;
constexpr int kSc1 = 16;  // buffer-load cache policy: agent-coherent (SC1)

__device__ __forceinline__ float act_fn(float g, float u, int kind, float beta, float lbeta) {
    if (kind == K3_ACT_SITU) {
        // beta*tanh(g/beta)*sigmoid(g) * lbeta*tanh(u/lbeta)   (ops.py:17-28)
        const float a = beta * tanhf(g / beta) / (1.0f + expf(-g));
        return a * (lbeta > 0.f ? lbeta * tanhf(u / lbeta) : u);
    }
    return g / (1.0f + expf(-g)) * u;  // silu(g) * u                 (ops.py:42-43)
}

__device__ __forceinline__ void store_coherent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_coherent(uint32_t *p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint4 load16_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1));
}

// Epoch of this launch: workspace word 0, read by thread 0 of every block into *lds
// (callers __syncthreads() before use).  Barrier j of a launch publishes epoch + j + 1.
// Once barrier 0 has passed, every block has read the epoch, and block 0 advances it by
// the kernel's barrier count (barrier_advance_epoch), so flag values keep increasing
// from launch to launch whatever the grid size of each launch.
__device__ __forceinline__ void barrier_epoch(uint32_t *ws, uint32_t *lds) {
    if (threadIdx.x == 0) *lds = __hip_atomic_load(ws, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void barrier_advance_epoch(uint32_t *ws, uint32_t epoch, uint32_t n_barriers) {
    if (blockIdx.x == 0 && threadIdx.x == 0) store_coherent(ws, epoch + n_barriers);
}

// Called by ONE whole wave, after its coherent data stores: wait for them to complete,
// publish `value` for this block, then wait (two-level) until every block has published.
// The caller follows with __syncthreads().  Loads the wave issued before this call are
// also waited for (vmcnt is in order), so the publishing wave should not be holding
// weight prefetches.
__device__ __forceinline__ void barrier_publish_and_wait(uint32_t *ws, uint32_t value) {
    uint32_t *flags = reinterpret_cast<uint32_t *>(reinterpret_cast<char *>(ws) + kFlagsOffset);
    uint32_t *gflags = reinterpret_cast<uint32_t *>(reinterpret_cast<char *>(ws) + kGroupFlagsOffset);
    const int nb = static_cast<int>(gridDim.x);
    const int G = nb < kGroups ? nb : kGroups;
    const int lane = threadIdx.x & 63;
    __builtin_amdgcn_s_waitcnt(0);
    if (lane == 0) store_coherent(flags + blockIdx.x, value);
    uint32_t spins = 0;
    auto timed_out = [&]() {
        __builtin_amdgcn_s_sleep(1);
        if (++spins > kSpinLimit) {
            if (lane == 0) store_coherent(ws + kErrWord, kErrBarrierTimeout);
            return true;
        }
        return false;
    };
    if (static_cast<int>(blockIdx.x) < G) {  // group leader: members g, g+G, g+2G, ...
        for (;;) {
            int behind = 0;
            for (int b = static_cast<int>(blockIdx.x) + G * lane; b < nb; b += 64 * G) {
                const uint32_t f = __hip_atomic_load(flags + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                behind |= static_cast<int32_t>(f - value) < 0;
            }
            if (!__any(behind) || timed_out()) break;
        }
        if (lane == 0) store_coherent(gflags + blockIdx.x * kGroupStride, value);
    }
    for (;;) {
        int behind = 0;
        if (lane < G) {
            const uint32_t f = __hip_atomic_load(gflags + lane * kGroupStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            behind = static_cast<int32_t>(f - value) < 0;
        }
        if (!__any(behind) || timed_out()) break;
    }
}

// Grid size such that every block is resident at once (required by the barrier).
int resident_blocks(const void *kernel, int block_threads, size_t lds_bytes, int *out);

}  // namespace k3
