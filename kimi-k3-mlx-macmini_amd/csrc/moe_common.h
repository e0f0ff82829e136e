// Pieces shared by the expert-FFN, MoE-layer and grouped kernels: the expert activations.
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

}  // namespace k3
