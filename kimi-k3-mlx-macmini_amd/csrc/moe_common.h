// Pieces shared by the expert-FFN, MoE-layer and grouped kernels: the expert activations
// and wave-uniform pointers read from the expert table.
#pragma once

#include "k3_common.h"

namespace k3 {

__device__ __forceinline__ float act_fn(float g, float u, int kind, float beta, float lbeta) {
    if (kind == K3_ACT_SITU) {
        // beta*tanh(g/beta)*sigmoid(g) * lbeta*tanh(u/lbeta)   (ops.py:17-28)
        const float a = beta * tanhf(g / beta) / (1.0f + expf(-g));
        return a * (lbeta > 0.f ? lbeta * tanhf(u / lbeta) : u);
    }
    return g / (1.0f + expf(-g)) * u;  // silu(g) * u                 (ops.py:42-43)
}

// A 64-bit pointer held in memory, made wave-uniform (SGPRs) so buffer resources built
// from it need no waterfall loop.
__device__ __forceinline__ const void *uniform_ptr(uint64_t p) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
    return reinterpret_cast<const void *>((static_cast<uint64_t>(hi) << 32) | lo);
}

}  // namespace k3
