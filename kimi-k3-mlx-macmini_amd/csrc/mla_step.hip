// One decode token through a whole MLA layer at batch 1: the projections on either side
// of the absorbed attention core, the latent-cache append and the output gate.
//
// Reference: MLAAttention.__call__ (air_llm/models/kimi_k3/attention_mla.py:168-216):
//   q   = rmsnorm(x @ q_a.T, q_a_layernorm) @ q_b.T                  -> [H, nope + rope]
//   ckv = x @ kv_a.T;  c_new = rmsnorm(ckv[:r], kv_a_layernorm);  r_new = ckv[r:]
//   cache.append(c_new, r_new)                                      (attention_mla.py:89-108)
//   o   = absorbed attention core over the cache                     (attention_mla.py:193-212)
//   o   = o * sigmoid(x @ g_proj.T)  (mla_use_output_gate);  out = o @ o_proj.T
//
// Seven stream-ordered launches, no host synchronisation:
//   S1  rows of q_a, kv_a and g_proj against x (one grid, three block ranges);
//   S2  rows of q_b against the normalised q_a output (every block normalises the 1536-wide
//       vector itself, so no launch is spent on it), and one block that normalises the kv
//       latent and writes the new cache row (bf16) at position pos;
//   core  the absorbed core of k3_mla_decode_absorbed (four launches) over the pos + 1
//       cache rows, its last launch multiplying o by sigmoid(gate) as it writes it;
//   S3  rows of o_proj against the gated o.
// The row launches are the dense row kernels of dense_rows.h.
#include <algorithm>

#include "dense_rows.h"

namespace k3 {
namespace {

size_t up256(size_t v) { return (v + 255) & ~size_t(255); }

struct StepWs {
    size_t qa, ckv, gl, q, o, core, total;
};

StepWs step_ws_layout(int64_t hidden, int64_t ql, int64_t H, int64_t nope, int64_t rope, int64_t v, int64_t r,
                      int64_t T) {
    StepWs L{};
    size_t off = 0;
    L.qa = off, off += up256(ql * 4);
    L.ckv = off, off += up256((r + rope) * 4);
    L.gl = off, off += up256(H * v * 4);
    L.q = off, off += up256(H * (nope + rope) * 4);
    L.o = off, off += up256(H * v * 4);
    L.core = off, off += static_cast<size_t>(k3_mla_workspace_size(H, T));
    L.total = off;
    (void)hidden;
    return L;
}

}  // namespace
}  // namespace k3

using namespace k3;

extern "C" int64_t k3_mla_step_workspace_size(int64_t hidden, int64_t q_lora_rank, int64_t heads, int64_t nope_dim,
                                              int64_t rope_dim, int64_t v_dim, int64_t kv_lora_rank, int64_t T) {
    return static_cast<int64_t>(
        step_ws_layout(hidden, q_lora_rank, heads, nope_dim, rope_dim, v_dim, kv_lora_rank, T).total);
}

extern "C" int k3_mla_step_decode(const void *x, int x_dtype, const void *q_a, const float *q_a_norm, const void *q_b,
                                  const void *kv_a, const float *kv_a_norm, const void *w_uk, const void *w_uv,
                                  const void *g_proj, const void *o_proj, void *lat, int64_t ld_lat, void *rot,
                                  int64_t ld_rot, int64_t cache_rows, int64_t pos, float eps, float scale, void *out,
                                  int out_dtype,
                                  int64_t hidden, int64_t q_lora_rank, int64_t heads, int64_t nope_dim,
                                  int64_t rope_dim, int64_t v_dim, int64_t kv_lora_rank, void *workspace,
                                  int64_t workspace_bytes, void *stream) {
    if (!x || !q_a || !q_a_norm || !q_b || !kv_a || !kv_a_norm || !w_uk || !w_uv || !o_proj || !lat || !rot || !out ||
        !workspace)
        return set_error(K3_ERR_NULL, "mla step: null pointer");
    if (x_dtype != K3_F32 && x_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "mla step: x_dtype %d", x_dtype);
    if (out_dtype != K3_F32 && out_dtype != K3_BF16) return set_error(K3_ERR_DTYPE, "mla step: out_dtype %d", out_dtype);
    const int64_t qhd = nope_dim + rope_dim, hv = heads * v_dim;
    if (hidden <= 0 || hidden % 8 || q_lora_rank <= 0 || q_lora_rank % 8 || hv <= 0 || hv % 8 ||
        hidden > kMaxWidth || q_lora_rank > kMaxWidth || hv > kMaxWidth || kv_lora_rank % 4 || rope_dim % 4)
        return set_error(K3_ERR_SHAPE, "mla step: hidden, q_lora_rank and heads*v must be multiples of 8, <= %d",
                         kMaxWidth);
    if (pos < 0 || pos >= cache_rows)
        return set_error(K3_ERR_SHAPE, "mla step: position %lld outside the cache's %lld rows", (long long)pos,
                         (long long)cache_rows);
    if (!aligned16(x) || !aligned16(q_a) || !aligned16(q_b) || !aligned16(kv_a) || !aligned16(o_proj) ||
        (g_proj && !aligned16(g_proj)) || !aligned16(q_a_norm) || !aligned16(kv_a_norm) || !aligned16(workspace))
        return set_error(K3_ERR_ALIGN, "mla step: vectors, weights and workspace must be 16-byte aligned");
    if (heads * qhd * q_lora_rank * 2 >= (1ll << 31) || hidden * hv * 2 >= (1ll << 31) ||
        q_lora_rank * hidden * 2 >= (1ll << 31))
        return set_error(K3_ERR_SHAPE, "mla step: a weight matrix exceeds 2 GiB");
    const int64_t T = pos + 1;
    const StepWs L = step_ws_layout(hidden, q_lora_rank, heads, nope_dim, rope_dim, v_dim, kv_lora_rank, T);
    if (workspace_bytes < static_cast<int64_t>(L.total))
        return set_error(K3_ERR_WORKSPACE, "mla step: workspace %lld < %zu bytes", (long long)workspace_bytes, L.total);
    char *ws = static_cast<char *>(workspace);
    float *qa = reinterpret_cast<float *>(ws + L.qa), *ckv = reinterpret_cast<float *>(ws + L.ckv);
    float *gl = reinterpret_cast<float *>(ws + L.gl), *q = reinterpret_cast<float *>(ws + L.q);
    float *o = reinterpret_cast<float *>(ws + L.o);
    auto st = static_cast<hipStream_t>(stream);
    // S1: q_a, kv_a, g_proj rows against x
    RowsArgs a{};
    a.x = x;
    a.x_bf16 = x_dtype == K3_BF16;
    a.K = static_cast<int>(hidden);
    a.w[0] = static_cast<const uint16_t *>(q_a), a.N[0] = static_cast<int>(q_lora_rank), a.y[0] = qa;
    a.w[1] = static_cast<const uint16_t *>(kv_a), a.N[1] = static_cast<int>(kv_lora_rank + rope_dim), a.y[1] = ckv;
    a.w[2] = static_cast<const uint16_t *>(g_proj), a.N[2] = g_proj ? static_cast<int>(hv) : 0, a.y[2] = gl;
    int rc = launch_rows<kModeX>(a, st);
    if (rc) return rc;
    // S2: q_b rows against the normalised q_a output; the cache row
    RowsArgs b{};
    b.src = qa, b.nw = q_a_norm, b.eps = eps, b.K = static_cast<int>(q_lora_rank);
    b.w[0] = static_cast<const uint16_t *>(q_b), b.N[0] = static_cast<int>(heads * qhd), b.y[0] = q;
    b.ckv = ckv, b.kvw = kv_a_norm;
    b.lat_row = static_cast<uint16_t *>(lat) + pos * ld_lat;
    b.rot_row = static_cast<uint16_t *>(rot) + pos * ld_rot;
    b.r = static_cast<int>(kv_lora_rank), b.rope = static_cast<int>(rope_dim), b.append = 1;
    rc = launch_rows<kModeNorm>(b, st);
    if (rc) return rc;
    // core over the pos + 1 cache rows
    rc = mla_decode_core(q, q + nope_dim, qhd, qhd, K3_F32, w_uk, w_uv, lat, ld_lat, rot, ld_rot, T, heads,
                         kv_lora_rank, rope_dim, nope_dim, v_dim, scale, o, K3_F32, v_dim, g_proj ? gl : nullptr,
                         ws + L.core, workspace_bytes - static_cast<int64_t>(L.core), stream);
    if (rc) return rc;
    // S3: o_proj rows against the gated o
    RowsArgs c{};
    c.o = o, c.gl = nullptr, c.K = static_cast<int>(hv);
    c.w[0] = static_cast<const uint16_t *>(o_proj), c.N[0] = static_cast<int>(hidden);
    c.out = out, c.out_bf16 = out_dtype == K3_BF16;
    return launch_rows<kModeGate>(c, st);
}
