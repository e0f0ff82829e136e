// Internal interface of the MXFP4 GEMV kernels (shared with the MoE kernels).
#pragma once

#include "k3_common.h"

namespace k3 {

struct GemvArgs {
    const void *x;       // [M, K] bf16 or fp32, row stride ldx elements
    int64_t ldx;
    const void *packed;  // [N, K/2] u8
    const void *scales;  // [N, K/32] u8
    void *out;           // [M, N] fp32 or bf16, row stride ldo elements
    int64_t ldo;
    int M;               // tokens in this launch (<= 4)
    int64_t N;
    int64_t K;
    int x_bf16;
    int out_bf16;
};

constexpr size_t kGemvMaxLds = 160 * 1024;

void gemv_default_cfg(int64_t N, int64_t K, int *rpw, int *gpl);
int gemv_token_tile(int64_t K, int x_bf16);  // tokens per launch (0: K too long)
int gemv_launch(const GemvArgs &a, int rpw, int gpl, hipStream_t st);
int gemv_validate(const void *x, int x_dtype, const void *packed, const void *scales,
                  const void *out, int out_dtype, int64_t M, int64_t N, int64_t K);

}  // namespace k3
