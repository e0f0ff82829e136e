/*
 * k3hip -- MI355X (gfx950) C-ABI for the MXFP4 expert / latent-MLA decode hot path.
 *
 * Every entry point:
 *   - takes raw device pointers, int64 sizes and a hipStream_t (passed as void*),
 *   - is asynchronous and stream-ordered (the caller synchronises),
 *   - allocates nothing: outputs and workspaces belong to the caller,
 *   - returns K3_OK (0) or a K3_ERR_* status; k3_last_error() gives the message for
 *     the calling thread.
 *
 * Layouts (all row-major, contiguous):
 *   packed  uint8 [N, K/2]   E2M1 codes, element 2i = low nibble of byte i
 *   scales  uint8 [N, K/32]  E8M0, 2^(b-127) for elements 32j..32j+31 of the row
 *   (air_llm/models/kimi_k3/mxfp4.py:3-11, k3ref/weights.py:26-37)
 */
#ifndef K3HIP_H
#define K3HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------------ */
#define K3_OK              0
#define K3_ERR_SHAPE       1  /* inconsistent / unsupported sizes (reference: ValueError) */
#define K3_ERR_DTYPE       2  /* unsupported dtype enum                                   */
#define K3_ERR_ALIGN       3  /* pointer not 16-byte aligned where a 128-bit path needs it */
#define K3_ERR_SCALE_RANGE 4  /* E8M0 bytes outside 2..252 (reference: ValueError)        */
#define K3_ERR_WORKSPACE   5  /* workspace too small                                      */
#define K3_ERR_HIP         6  /* a HIP launch / runtime call failed                      */
#define K3_ERR_NULL        7  /* required pointer is NULL                                 */

/* ---- dtype enums ------------------------------------------------------------------- */
#define K3_F32   0
#define K3_BF16  1

/* ---- activation enums (expert FFN) ------------------------------------------------- */
#define K3_ACT_SILU  0   /* silu(g) * u                         (air_llm/models/kimi_k3/ops.py:42-43) */
#define K3_ACT_SITU  1   /* b*tanh(g/b)*sigmoid(g) * bl*tanh(u/bl) (air_llm/models/kimi_k3/ops.py:17-28) */

/* ---- router enums ------------------------------------------------------------------ */
#define K3_ROUTE_SOFTMAX      0  /* softmax(logits); top-k in probability order (selected on the
                                    logits, which order exactly as the probabilities do)  */
#define K3_ROUTE_SIGMOID_BIAS 1  /* sigmoid(logits); select on +bias; weights from raw (moe.py:65-76) */

const char *k3_last_error(void);
const char *k3_version(void);

/* Bit-exact dequantisation to fp32 (out_dtype K3_F32) or bf16 (K3_BF16), [N, K].
 * Replaces decode_mxfp4_mlx (air_llm/models/kimi_k3/mxfp4.py:68-81) with the values of
 * k3ref.weights.decode_mxfp4 (k3ref/weights.py:29-37) for every code and scale byte. */
int k3_mxfp4_decode(const void *packed, const void *scales, void *out, int out_dtype,
                    int64_t N, int64_t K, void *stream);

/* Device-side min and max of n E8M0 bytes into minmax[0], minmax[1] (int32).
 * Backs assert_scales_representable (air_llm/models/kimi_k3/mxfp4.py:58-65). */
int k3_scale_minmax(const void *scales, int64_t n, int32_t *minmax, void *stream);

/* Fused MXFP4 matvec / small-M matmul: out[M, N] = x[M, K] @ W^T, W given by
 * (packed, scales), weights decoded in registers, fp32 accumulation.
 * x_dtype K3_F32 or K3_BF16; out_dtype K3_F32 (the reference kernel's output) or K3_BF16
 * (round-to-nearest-even of the fp32 accumulator).
 * Replaces mxfp4_matvec_fused (air_llm/kernels/metal/mxfp4_matvec.py:75-96) and the
 * Metal kernel body (air_llm/kernels/metal/mxfp4_matvec.py:29-63). */
int k3_mxfp4_matvec(const void *x, int x_dtype, const void *packed, const void *scales,
                    void *out, int out_dtype, int64_t M, int64_t N, int64_t K, void *stream);

/* ---- MoE expert FFN ---------------------------------------------------------------- */

/* Workspace bytes k3_expert_ffn needs for intermediate size I (the fp32 act vector passed
 * between its two launches).  Needs no initialisation.  Calls that share a workspace must
 * not overlap (calls on one stream never do). */
int64_t k3_expert_ffn_workspace_size(int64_t I);

/* One routed expert at batch 1, two stream-ordered launches (gate/up + act, then the down
 * GEMV): out[H] = act(x Wg^T, x Wu^T) Wd^T with gate/up packed [I, H/2] / scales [I, H/32]
 * and down packed [H, I/2] / scales [H, I/32].
 * act_kind K3_ACT_SILU (beta ignored) or K3_ACT_SITU (linear_beta <= 0 means None).
 * H and I must be multiples of 128, H <= 8192.
 * Replaces LatentMoE.expert_forward (air_llm/models/kimi_k3/moe.py:90-103) with the
 * k3ref semantics (k3ref/layers.py:226-234). */
int k3_expert_ffn(const void *x, int x_dtype, const void *gate_packed, const void *gate_scales,
                  const void *up_packed, const void *up_scales, const void *down_packed,
                  const void *down_scales, void *out, int out_dtype, int64_t H, int64_t I,
                  int act_kind, float beta, float linear_beta, void *workspace,
                  int64_t workspace_bytes, void *stream);

/* k3_expert_ffn without a caller workspace and without any allocation: for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  act lives in a
 * static device array of 16384 fp32 values (64 KiB per GPU, held until the process ends);
 * I > 16384 returns K3_ERR_WORKSPACE.  Every call on a GPU shares that array, so calls that
 * overlap on one GPU (on different streams, or from different threads without ordering)
 * race; calls on one stream never overlap.  Same results as k3_expert_ffn. */
int k3_expert_ffn_noalloc(const void *x, int x_dtype, const void *gate_packed, const void *gate_scales,
                          const void *up_packed, const void *up_scales, const void *down_packed,
                          const void *down_scales, void *out, int out_dtype, int64_t H, int64_t I,
                          int act_kind, float beta, float linear_beta, void *stream);

/* ---- routed MoE layer at batch 1 ------------------------------------------------------ */

/* Workspace bytes for k3_moe_layer_decode / k3_moe_route (pass shared_I = 0 without a
 * shared expert).  Its first 4096 bytes hold arrival counters (finished router blocks,
 * finished blocks of each range of output rows; at that place for every shape): zero-fill
 * them before the first call; every call returns them to zero.  The rest is rewritten by every call.  Calls that share a workspace must not
 * overlap (calls on one stream never do). */
int64_t k3_moe_layer_workspace_size(int64_t H, int64_t I, int64_t shared_I, int64_t n_experts,
                                    int64_t top_k);

/* Byte offsets of the workspace's records: [0] logits[E] f32, [1] scores[E] f32 (softmax
 * probabilities or raw sigmoid scores), [2] corrected scores[E] f32, [3] top-k expert ids
 * int32[k], [4] top-k weights f32[k], [5] shared act, [6] routed act, [7] shared output.
 * The RouterResult of LatentMoE.route (air_llm/models/kimi_k3/moe.py:32-37) is read there. */
int k3_moe_layer_workspace_offsets(int64_t H, int64_t I, int64_t shared_I, int64_t n_experts,
                                   int64_t top_k, int64_t *offsets);

/* Router + top-k only (LatentMoE.route, air_llm/models/kimi_k3/moe.py:65-76 and
 * k3ref/layers.py:214-224): router_w bf16 [E, H]; route_kind K3_ROUTE_SOFTMAX or
 * K3_ROUTE_SIGMOID_BIAS (router_bias f32 [E] added for selection only); weights gathered
 * from the raw scores, divided by (sum + 1e-20) when renormalize and top_k > 1, times
 * scaling.  Ties go to the lower expert index; softmax selects on the logits (the
 * probabilities' order without fp32 rounding ties), and a NaN or infinite logit makes every
 * probability NaN and selects the k lowest indices.  Results land in the workspace records.
 * Resets the router's arrival counter itself (one small launch before the router rows), so
 * it routes correctly whatever the workspace's counter bytes hold. */
int k3_moe_route(const void *x, int x_dtype, const void *router_w, const void *router_bias,
                 int route_kind, int renormalize, float scaling, int64_t H, int64_t n_experts,
                 int64_t top_k, void *workspace, int64_t workspace_bytes, void *stream);

/* Selection half of the router for T tokens at once, from router logits computed by the
 * caller (fp32 [T, E], row stride ld_logits; the prefill path takes them from one GEMM over
 * all tokens): per token, scores = softmax or sigmoid of the logits, selection on the logits
 * for softmax (the probabilities' order) and on scores + router_bias for
 * K3_ROUTE_SIGMOID_BIAS, exact top-k with ties to the lower expert index,
 * weights gathered from the raw scores, divided by (sum + 1e-20) when renormalize and
 * top_k > 1, times scaling.  Outputs: expert_idx int32 [T, top_k] (largest first),
 * expert_w f32 [T, top_k], scores and corrected f32 [T, E].  One block per token.
 * Replaces the per-token selection of LatentMoE.route (air_llm/models/kimi_k3/moe.py:67-76;
 * k3ref/layers.py:214-224), whose logits are one matmul over the flattened tokens. */
int k3_moe_topk(const float *logits, int64_t ld_logits, int64_t T, int64_t n_experts,
                const float *router_bias, int route_kind, int renormalize, float scaling, int64_t top_k,
                int32_t *expert_idx, float *expert_w, float *scores, float *corrected, void *stream);

/* Whole routed MoE layer for one token: route (as k3_moe_route), then
 *   out[H] = shared(x) + sum_j w_j * expert_{idx_j}(x)
 * with no device-to-host synchronisation.  expert_table is a device array of
 * n_experts x 6 uint64 pointers (gate packed, gate scales, up packed, up scales, down
 * packed, down scales) in the k3_expert_ffn layouts, so every expert stays resident and
 * each selected expert is read once.  shared_gate/up bf16 [shared_I, H] and shared_down
 * bf16 [H, shared_I] are optional (all NULL: no shared expert).  top_k <= 16,
 * n_experts <= 1024, H/I/shared_I multiples of 128.
 * Replaces LatentMoE.__call__ / expert_forward / shared_forward
 * (air_llm/models/kimi_k3/moe.py:90-132; k3ref/layers.py:226-261) without the K3
 * latent down/norm/up wrapper. */
int k3_moe_layer_decode(const void *x, int x_dtype, const void *router_w, const void *router_bias,
                        int route_kind, int renormalize, float scaling, const void *expert_table,
                        const void *shared_gate, const void *shared_up, const void *shared_down,
                        void *out, int out_dtype, int64_t H, int64_t I, int64_t shared_I,
                        int64_t n_experts, int64_t top_k, int act_kind, float beta,
                        float linear_beta, void *workspace, int64_t workspace_bytes, void *stream);

/* ---- grouped routed experts for many tokens (prefill) ------------------------------------ */

/* Workspace bytes k3_moe_grouped_ffn needs (grouping records, the E4M3 terms of x and of the
 * activations of every routed pair with their E8M0 scales, fp32 per-pair expert outputs).
 * No initialisation. */
int64_t k3_moe_grouped_workspace_size(int64_t T, int64_t top_k, int64_t n_experts, int64_t H, int64_t I);

/* y[t] = sum_j w[t, j] * expert_{idx[t, j]}(x[t]) for T tokens at once:
 *   x [T, H] bf16 or fp32 (x_dtype); expert_idx int32 [T, top_k] (every id in 0..n_experts-1); expert_w f32
 *   [T, top_k]; expert_table as in k3_moe_layer_decode (packed pointers 16-byte aligned,
 *   scale pointers 2-byte aligned, E8M0 bytes 2..252); out [T, H] f32 or bf16.
 * The (token, slot) pairs are grouped by expert on the device and each expert runs as a
 * GEMM with M = its token count on native MXFP4 MFMA (v_mfma_scale_f32_16x16x128_f8f6f4:
 * the weights as stored, bf16 x as two E4M3 terms (exact), fp32 x and the activation as
 * three (about 12 bits), all with E8M0
 * scales per 32), so each expert's weights are read once per 64-token tile.  Normwise error
 * about 1e-4 of fp64 (the MFMA's own accumulation).  Deterministic.  H and I must be
 * multiples of 64.
 * Replaces the per-expert dispatch loop of LatentMoE.__call__
 * (air_llm/models/kimi_k3/moe.py:110-132; k3ref/layers.py:241-261) for prefill. */
int k3_moe_grouped_ffn(const void *x, int x_dtype, const int32_t *expert_idx, const float *expert_w,
                       const void *expert_table, void *out, int out_dtype, int64_t T, int64_t H,
                       int64_t I, int64_t n_experts, int64_t top_k, int act_kind, float beta,
                       float linear_beta, void *workspace, int64_t workspace_bytes, void *stream);

/* ---- routed experts for a few decode tokens, each selected expert read once ---------------- */

/* Workspace bytes k3_moe_routed_decode needs for T tokens (the union records, fp32 act and
 * down-row totals per (token, slot) pair).  No initialisation: every call rewrites what it
 * reads. */
int64_t k3_moe_routed_workspace_size(int64_t T, int64_t H, int64_t I, int64_t n_experts, int64_t top_k);

/* y[t] = sum_j w[t, j] * expert_{idx[t, j]}(x[t]) for T <= 8 decode tokens, with each expert
 * any token selects read from HBM once for all the tokens routed to it:
 *   x [T, H] bf16 or fp32 (x_dtype); expert_idx int32 [T, top_k]; expert_w f32 [T, top_k];
 *   expert_table as in k3_moe_layer_decode; out [T, H] f32 or bf16.
 * A token is gathered once per expert, with the weight of its first slot holding it; ids
 * outside 0..n_experts-1 contribute nothing.  Four stream-ordered launches (the union of the
 * routed experts on the device, the gate/up rows of every union expert against its tokens,
 * its down rows, a fixed-order combine), no host synchronisation, fp32 accumulation,
 * deterministic.  H and I multiples of 128, H <= 8192, I <= 4096, top_k <= 16,
 * n_experts <= 1024.
 * Replaces the per-expert dispatch loop of LatentMoE.__call__ (air_llm/models/kimi_k3/moe.py:
 * 119-127, h[ti] gathered per expert; k3ref/layers.py:241-261) at decode batch sizes, whose
 * kernel takes the M tokens of an expert in one launch (mxfp4_matvec.py:89-95). */
int k3_moe_routed_decode(const void *x, int x_dtype, const int32_t *expert_idx, const float *expert_w,
                         const void *expert_table, void *out, int out_dtype, int64_t T, int64_t H,
                         int64_t I, int64_t n_experts, int64_t top_k, int act_kind, float beta,
                         float linear_beta, void *workspace, int64_t workspace_bytes, void *stream);

/* Workspace bytes for k3_moe_layer_decode_multi (the k3_moe_routed_decode records plus the
 * router records and the shared expert's act and output for T tokens).  No initialisation. */
int64_t k3_moe_layer_multi_workspace_size(int64_t T, int64_t H, int64_t I, int64_t shared_I,
                                          int64_t n_experts, int64_t top_k);

/* Byte offsets of k3_moe_layer_decode_multi's router records: [0] logits f32 [T, E], [1] scores
 * f32 [T, E] (softmax probabilities or raw sigmoid scores), [2] corrected scores f32 [T, E],
 * [3] top-k expert ids int32 [T, k], [4] top-k weights f32 [T, k] (the RouterResult of
 * LatentMoE.route, air_llm/models/kimi_k3/moe.py:32-37, for the T tokens). */
int k3_moe_layer_multi_workspace_offsets(int64_t T, int64_t H, int64_t I, int64_t shared_I,
                                         int64_t n_experts, int64_t top_k, int64_t *offsets);

/* k3_moe_layer_decode for T <= 8 decode tokens at once, x [T, H] and out [T, H]: the router
 * rows and the shared gate/up rows against all T tokens in one launch (bf16 rows, exact
 * products, fp32 accumulation), the batched top-k (as k3_moe_topk), the routed experts as in
 * k3_moe_routed_decode (every expert any token selects read once for all the tokens routed to
 * it), the shared down rows, and the fixed-order combine with the shared output: six or seven
 * launches, no host synchronisation.  The shared expert's gate/up and down rows run on a
 * library-owned side stream of the current device, forked from `stream` at the start of the
 * call and joined to it before the routed down launch through events (as
 * k3_moe_latent_layer_decode_multi, which joins before the up projection);
 * without it (K3HIP_SIDE_STREAM=0 in the environment, a first call made under capture, or a
 * call under capture while another capture on the device holds the capture side stream) the
 * gate/up rows run with the router rows and the down rows as extra blocks of the routed down
 * launch (when the T act rows fit 32 KB and shared_I <= 4096, else a launch of their own).
 * Arguments as k3_moe_layer_decode, plus T;
 * shared_I a multiple of 128, <= 8192.
 * Replaces LatentMoE.__call__ (air_llm/models/kimi_k3/moe.py:110-132, without the latent
 * wrapper) for a decode batch of T tokens, whose dispatch loop gathers every token routed to
 * an expert (h[ti], moe.py:120-124) and whose kernel takes M tokens per launch
 * (mxfp4_matvec.py:89-95). */
int k3_moe_layer_decode_multi(const void *x, int x_dtype, const void *router_w, const void *router_bias,
                              int route_kind, int renormalize, float scaling, const void *expert_table,
                              const void *shared_gate, const void *shared_up, const void *shared_down,
                              void *out, int out_dtype, int64_t T, int64_t H, int64_t I, int64_t shared_I,
                              int64_t n_experts, int64_t top_k, int act_kind, float beta, float linear_beta,
                              void *workspace, int64_t workspace_bytes, void *stream);

/* Workspace bytes for k3_moe_latent_layer_decode_multi (the T-token records of
 * k3_moe_layer_decode_multi with the routed part at the latent width, plus the latent state
 * and routed sum [T, latent]).  No initialisation. */
int64_t k3_moe_latent_layer_multi_workspace_size(int64_t T, int64_t H, int64_t latent, int64_t I,
                                                 int64_t shared_I, int64_t n_experts, int64_t top_k);

/* Byte offsets of k3_moe_latent_layer_decode_multi's router records, in the order of
 * k3_moe_layer_multi_workspace_offsets. */
int k3_moe_latent_layer_multi_workspace_offsets(int64_t T, int64_t H, int64_t latent, int64_t I,
                                                int64_t shared_I, int64_t n_experts, int64_t top_k,
                                                int64_t *offsets);

/* k3_moe_latent_layer_decode for T <= 8 decode tokens at once, x [T, H], out [T, H]: the
 * router, latent down and shared gate/up rows against all T tokens in one launch, the batched
 * sigmoid + bias top-k, the routed experts on h at the latent width as in
 * k3_moe_routed_decode (every selected expert read once for all its tokens), the shared down
 * rows, and the up projection rows against rmsnorm(routed sum) * latent_norm with the shared
 * output added: eight launches, no host synchronisation.  The shared expert's gate/up and
 * down rows run on a library-owned side stream of the current device (one for calls under
 * capture, one for the rest, created on the first call, default priority), forked from `stream` at the start of the call and joined to it
 * before the up projection through events, so the call stays ordered on `stream` and can be
 * captured in a graph (a first call made under capture, a call under capture while another
 * capture on the device holds the capture side stream, or K3HIP_SIDE_STREAM=0 in the
 * environment, runs them on `stream`).  Arguments as
 * k3_moe_latent_layer_decode, plus T; shared_I a multiple of 128, <= 8192.
 * Replaces LatentMoE.__call__ (air_llm/models/kimi_k3/moe.py:110-132) for a decode batch of T
 * tokens, including the latent down/norm/up wrapper (moe.py:116,129-130). */
int k3_moe_latent_layer_decode_multi(const void *x, int x_dtype, const void *router_w, const void *router_bias,
                                     int renormalize, float scaling, const void *expert_table,
                                     const void *latent_down, const void *latent_up, const void *latent_norm,
                                     float eps, const void *shared_gate, const void *shared_up,
                                     const void *shared_down, void *out, int out_dtype, int64_t T, int64_t H,
                                     int64_t latent, int64_t I, int64_t shared_I, int64_t n_experts,
                                     int64_t top_k, int act_kind, float beta, float linear_beta, void *workspace,
                                     int64_t workspace_bytes, void *stream);

/* Workspace bytes for k3_moe_latent_layer_decode: the k3_moe_layer_decode records plus the
 * bf16 latent state and the fp32 routed sum.  Same counter rule as k3_moe_layer_workspace_size
 * (first 4096 bytes zero before the first call; every call returns them to zero). */
int64_t k3_moe_latent_layer_workspace_size(int64_t H, int64_t latent, int64_t I, int64_t shared_I,
                                           int64_t n_experts, int64_t top_k);

/* K3's routed layer with its latent wrapper for one token (x [H], bf16 or fp32 by x_dtype):
 *   route (sigmoid + bias, as k3_moe_route) on x;
 *   h = latent_down . x                               latent_down bf16 [latent, H]; h is rounded
 *                                                     to bf16 for a bf16 x (the reference's bf16
 *                                                     matmul) and stays fp32 for an fp32 x
 *   y = sum_j w_j * expert_{idx_j}(h)                 experts of width latent (expert_table)
 *   out = latent_up . (latent_norm * y / sqrt(mean(y^2) + eps)) + shared(x)
 * latent_up bf16 [H, latent], latent_norm fp32 [latent]; shared_* as in k3_moe_layer_decode
 * (K3's two shared experts are one MLP of width shared_I).  Four stream-ordered launches,
 * no device-to-host synchronisation.  latent, I, shared_I multiples of 128, H <= 8192,
 * top_k <= 16, n_experts <= 1024.
 * Replaces LatentMoE.__call__ (air_llm/models/kimi_k3/moe.py:110-132) at batch 1, including
 * the latent down/norm/up wrapper (moe.py:116,129-130). */
int k3_moe_latent_layer_decode(const void *x, int x_dtype, const void *router_w, const void *router_bias, int renormalize,
                               float scaling, const void *expert_table, const void *latent_down,
                               const void *latent_up, const void *latent_norm, float eps,
                               const void *shared_gate, const void *shared_up, const void *shared_down,
                               void *out, int out_dtype, int64_t H, int64_t latent, int64_t I,
                               int64_t shared_I, int64_t n_experts, int64_t top_k, int act_kind, float beta,
                               float linear_beta, void *workspace, int64_t workspace_bytes, void *stream);

/* ---- latent-MLA absorbed decode (one query token, batch 1) ------------------------------ */

/* Workspace bytes k3_mla_decode_absorbed needs for H heads over T cached tokens (qa
 * hi/lo rows, one (ctx, max, sum) record per head per token split, and the W_UV products
 * of the four column quarters for v up to 1024).  No initialisation. */
int64_t k3_mla_workspace_size(int64_t H, int64_t T);

/* o[h] = W_UV[h] @ (softmax_t(scale * (q_nope[h] W_UK[h] . lat[t] + q_rot[h] . rot[t])) @ lat)
 * for every head h, over the T valid cache rows.
 *   q_nope [H, nope] rows ld_q elements apart, q_rot [H, rope] rows ld_q_rot apart
 *   (q_dtype K3_BF16 / K3_F32, the same for both)
 *   w_uk [H, nope, r], w_uv [H, v, r]: bf16, the two halves of kv_b (attention_mla.py:155-158)
 *   lat [T, r] rows ld_lat apart, rot [T, rope] rows ld_rot apart: the bf16 latent cache
 *   out [H, v] rows ld_out apart, out_dtype K3_F32 / K3_BF16
 * kv_lora_rank must be 512 and rope_dim 64 (Kimi-K3 and the benchmark shapes); nope <= 256;
 * v <= 1024; ld_lat and ld_rot multiples of 8; T >= 1.  fp32 accumulation, fp32
 * softmax, deterministic.
 * Replaces the absorbed attention core of MLAAttention.__call__
 * (air_llm/models/kimi_k3/attention_mla.py:193-212) for T == 1. */
int k3_mla_decode_absorbed(const void *q_nope, const void *q_rot, int64_t ld_q, int64_t ld_q_rot,
                           int q_dtype, const void *w_uk, const void *w_uv, const void *lat, int64_t ld_lat,
                           const void *rot, int64_t ld_rot, int64_t T, int64_t H,
                           int64_t kv_lora_rank, int64_t rope_dim, int64_t nope_dim, int64_t v_dim,
                           float scale, void *out, int out_dtype, int64_t ld_out, void *workspace,
                           int64_t workspace_bytes, void *stream);

/* k3_mla_decode_absorbed over an fp32 latent cache (the reference's default cache dtype,
 * MLACache with mx.float32, attention_mla.py:164; its view, :83-87): lat [T, r] and rot
 * [T, rope] fp32 rows ld_lat / ld_rot elements apart (multiples of 4).  Every other argument,
 * the workspace size included, as k3_mla_decode_absorbed.  The rows are read once, each split
 * on the device into two bf16 planes (hi = rne(v), lo = rne(v - hi)) whose four products with
 * the hi/lo query terms are all kept, so the fp32 cache enters to ~2^-16 relative.
 * Replaces the absorbed core of MLAAttention.__call__ (attention_mla.py:193-212) for T == 1
 * with the reference's fp32 cache. */
int k3_mla_decode_absorbed_f32(const void *q_nope, const void *q_rot, int64_t ld_q, int64_t ld_q_rot,
                               int q_dtype, const void *w_uk, const void *w_uv, const void *lat, int64_t ld_lat,
                               const void *rot, int64_t ld_rot, int64_t T, int64_t H,
                               int64_t kv_lora_rank, int64_t rope_dim, int64_t nope_dim, int64_t v_dim,
                               float scale, void *out, int out_dtype, int64_t ld_out, void *workspace,
                               int64_t workspace_bytes, void *stream);

/* ---- one decode token through a whole MLA layer (batch 1) ------------------------------ */

/* Workspace bytes k3_mla_step_decode needs (its projections' outputs and the attention
 * core's workspace for T = pos + 1 cache rows).  No initialisation. */
int64_t k3_mla_step_workspace_size(int64_t hidden, int64_t q_lora_rank, int64_t heads, int64_t nope_dim,
                                   int64_t rope_dim, int64_t v_dim, int64_t kv_lora_rank, int64_t T);

/* MLAAttention.__call__ for one token (air_llm/models/kimi_k3/attention_mla.py:168-216):
 *   q = rmsnorm(x q_a^T, q_a_norm) q_b^T; ckv = x kv_a^T; the cache row pos gets
 *   bf16(rmsnorm(ckv[:r], kv_a_norm)) and bf16(ckv[r:]) (MLACache.append,
 *   attention_mla.py:89-108); o = the absorbed core over rows 0..pos
 *   (k3_mla_decode_absorbed); o *= sigmoid(x g_proj^T) when g_proj is not null;
 *   out = o o_proj^T.
 * x [hidden] bf16 or fp32; q_a [q_lora_rank, hidden], q_b [heads*(nope+rope), q_lora_rank],
 * kv_a [r + rope, hidden], g_proj [heads*v, hidden] (or null), o_proj [hidden, heads*v]: bf16
 * row-major; q_a_norm [q_lora_rank], kv_a_norm [r]: fp32; w_uk / w_uv as for
 * k3_mla_decode_absorbed; lat / rot the bf16 cache with cache_rows rows (pos < cache_rows).
 * hidden, q_lora_rank and heads*v: multiples of 8, <= 12288.  fp32 accumulation and
 * norms.  Seven stream-ordered launches. */
int k3_mla_step_decode(const void *x, int x_dtype, const void *q_a, const float *q_a_norm, const void *q_b,
                       const void *kv_a, const float *kv_a_norm, const void *w_uk, const void *w_uv,
                       const void *g_proj, const void *o_proj, void *lat, int64_t ld_lat, void *rot,
                       int64_t ld_rot, int64_t cache_rows, int64_t pos, float eps, float scale, void *out,
                       int out_dtype, int64_t hidden, int64_t q_lora_rank, int64_t heads, int64_t nope_dim,
                       int64_t rope_dim, int64_t v_dim, int64_t kv_lora_rank, void *workspace,
                       int64_t workspace_bytes, void *stream);

/* ---- Kimi Delta Attention recurrent step (one token) -------------------------------------- */

/* For every value head h (q/k head h / (v_heads / qk_heads)), on the fp32 state
 * S [v_heads, key_dim, value_dim] in place:
 *   S[h] = S[h] * exp(g[h])[:, None];  S[h] += (beta[h] k) (x) (v[h] - k . S[h]);
 *   out[h] = (scale q) . S[h]
 * q, k [qk_heads, key_dim], v [v_heads, value_dim], g [v_heads, key_dim], beta [v_heads]:
 * in_dtype (K3_F32 / K3_BF16) for all five; out [v_heads, value_dim] out_dtype.  key_dim
 * must be 128 (K3's KDA heads), value_dim a multiple of 32.  fp32 arithmetic, fixed
 * reduction order.  Replaces one step of KDAAttention._recurrent
 * (air_llm/models/kimi_k3/attention_kda.py:65-90; naive_recurrent_kda,
 * k3ref/_vendor/kda_naive.py:46-60). */
int k3_kda_recurrent_decode(const void *q, const void *k, const void *v, const void *g, const void *beta,
                            int in_dtype, float *state, void *out, int out_dtype, int64_t qk_heads,
                            int64_t v_heads, int64_t key_dim, int64_t value_dim, float scale, void *stream);

/* T tokens in order through the same recurrence in one launch (a prefill, or several
 * decode tokens): q, k [T, qk_heads, key_dim], v [T, v_heads, value_dim], g [T, v_heads,
 * key_dim], beta [T, v_heads], out [T, v_heads, value_dim].  Each block keeps its state
 * columns in registers across the tokens, so the state is read and written once.
 * Replaces the token loop of KDAAttention._recurrent (attention_kda.py:73-90). */
int k3_kda_recurrent(const void *q, const void *k, const void *v, const void *g, const void *beta, int in_dtype,
                     float *state, void *out, int out_dtype, int64_t T, int64_t qk_heads, int64_t v_heads,
                     int64_t key_dim, int64_t value_dim, float scale, void *stream);

/* Workspace bytes k3_kda_step_decode needs for `heads` heads of 128 (projection outputs and
 * the recurrence output).  No initialisation. */
int64_t k3_kda_step_workspace_size(int64_t heads);

/* KDAAttention.__call__ for one token at batch 1 (air_llm/models/kimi_k3/attention_kda.py:94-115):
 *   q, k, v = silu(short_conv(x W^T)) with the convolution state (ops.py:46-60); q, k L2-normalised
 *   per head (eps 1e-6); g = gate_lower_bound * sigmoid(exp(A_log[h]) * (f_b(f_a x) + dt_bias));
 *   beta = sigmoid(b x); the recurrence of k3_kda_recurrent_decode on `state` (in place) with
 *   scale 128^-0.5; o = gated_rmsnorm(o, o_norm, g_proj x) per head (ops.py:36-39); out = o o_proj^T.
 * q/k/v/g_proj [heads*128, hidden], o_proj [hidden, heads*128], f_a [128, hidden],
 * f_b [heads*128, 128], b_proj [heads, hidden]: bf16.  q/k/v_conv [heads*128, conv_size],
 * o_norm [128], A_log [>= heads], dt_bias [heads*128]: fp32.  conv_in / conv_out
 * [3, conv_size - 1, heads*128] fp32 (q, k, v; oldest input first): distinct buffers, conv_out
 * receives the shifted window.  head_dim must be 128; heads*128 and hidden <= 12288.
 * Four stream-ordered launches. */
int k3_kda_step_decode(const void *x, int x_dtype, const void *q_proj, const void *k_proj, const void *v_proj,
                       const void *g_proj, const void *o_proj, const void *f_a, const void *f_b, const void *b_proj,
                       const float *q_conv, const float *k_conv, const float *v_conv, const float *conv_in,
                       float *conv_out, const float *o_norm, const float *A_log, const float *dt_bias, float *state,
                       void *out, int out_dtype, int64_t hidden, int64_t heads, int64_t head_dim, int64_t conv_size,
                       float gate_lower_bound, float eps, void *workspace, int64_t workspace_bytes, void *stream);

/* ---- HBM calibration ------------------------------------------------------------------- */

/* Streaming read of `bytes` (multiple of 16) from src; sink is a >= 4096-byte device scratch
 * word array that keeps the loads live.  No counterpart in the reference: the benchmark's
 * measured bandwidth ceiling for one launch of a given size, and the known-size kernel the
 * profiler's FETCH_SIZE counter is scaled by. */
int k3_stream_read(const void *src, int64_t bytes, void *sink, void *stream);

/* Streaming copy of `bytes` (multiple of 16) from src to dst.  No counterpart in the
 * reference: the known-size kernel the profiler's WRITE_SIZE counter is scaled by. */
int k3_stream_copy(void *dst, const void *src, int64_t bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* K3HIP_H */
