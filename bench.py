"""Benchmark: MXFP4 expert GEMV GB/s (% of HBM peak) and us per MoE layer at batch 1.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--workloads expert,layer,...]

One JSON line on stdout.  The headline workload is one SwiGLU expert at batch 1
(hidden 7168, intermediate 2048, MXFP4 weights with E8M0 scales in [118, 130], bf16 x):
a step is one expert FFN (a gate/up + activation launch, then the down GEMV) on a different
resident expert (64 experts rotate, 1.5 GB, so the 256 MB MALL cannot serve the weights).
`value` is algorithmic weight bytes per second over the K timed steps; `roofline` is that
step's (its two launches) and `cpu_baseline` a torch-CPU restatement of the k3ref path
timed on a bounded sample on this host.  The same line carries, as sub-objects:
  moe_layer          384 resident experts, top-8 softmax routing, a bf16 shared expert,
                     a fresh token per step;
  k3_latent_layer    K3's routed layer with its latent wrapper (896 experts, top-16);
  checkpoint_ingest  host-to-HBM ingest of K3-shaped experts from safetensors shards;
  moe_prefill        2048 tokens x top-8 on the grouped MXFP4-MFMA path, Zipf(1.1) load;
  gemv               one [2048 x 7168] projection;
  mla_decode         the absorbed MLA core, 64 heads over 32768 cached tokens;
  mla_step           one token through a whole MLA layer at K3 shapes;
  kda_decode         one KDA recurrent step (96 heads of 128 x 128 fp32 state), and a
                     256-token prefill through the recurrence in one launch;
  kda_step           one token through a whole KDA layer at K3 shapes, and a 256-token
                     prompt through its prefill path;
  read_ceiling       single streaming-read / copy launches of the same byte counts.
`cpu_baseline` also times the 384-expert layer and the MLA core on the CPU (moe_layer,
mla_decode sub-objects).

Synthetic, seeded data; weights are random-init with the benchmark shapes.  Steps are
captured once into a HIP graph and replayed, so the timed region is GPU work plus the
graph's launch gaps, without Python launch overhead.  `--gpus N` with N > 1 exits: k3hip
has no multi-GPU path.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "kimi-k3-mlx-macmini_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0           # MI355X HBM3E, published
H, I = 7168, 2048
E_LAYER, TOPK = 384, 8
ROTATE = 64                     # distinct experts cycled by the expert / GEMV benches

METRIC = "MXFP4 expert GEMV GB/s (% of HBM peak); us per MoE layer at batch 1"


def proj_bytes(n, k):
    return n * k // 2 + n * k // 32


EXPERT_BYTES = 2 * proj_bytes(I, H) + proj_bytes(H, I)          # 23,396,352
EXPERT_IO = H * 2 + H * 4                                        # x bf16 in, y fp32 out
LAYER_BYTES = E_LAYER * H * 2 + TOPK * EXPERT_BYTES + 3 * H * I * 2   # 280,756,224
GEMV_BYTES = proj_bytes(I, H) + H * 2 + I * 2                     # 7,817,216


def rand_mxfp4(torch, gen, n, k, device):
    p = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=device, generator=gen)
    s = torch.randint(118, 131, (n, k // 32), dtype=torch.uint8, device=device, generator=gen)
    return p, s


EAGER = False                   # --eager: launch every step directly (profiler counter runs)


def graph_time(torch, fn, steps, warmup):
    """Capture `steps` calls of fn(i) into one graph and replay it; also replay a graph of
    `warmup` calls first.  Returns seconds for the timed replay (synchronised both sides).
    With --eager the steps are launched one by one instead (for per-dispatch profiler
    counters); the timing then includes the host launch path."""
    stream = torch.cuda.current_stream()
    for i in range(3):
        fn(i)
    torch.cuda.synchronize()
    if EAGER:
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(steps):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3, time.perf_counter() - t0
    if warmup:
        gw = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gw):
            for i in range(warmup):
                fn(i)
        gw.replay()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            fn(i)
    torch.cuda.synchronize()
    g.replay()                      # first replay pays one-time costs
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return e0.elapsed_time(e1) / 1e3, wall


def step_stats(torch, fn, chunk=64, reps=16):
    """Per-step time distribution: a graph of `chunk` calls (a whole expert / cache rotation)
    replayed `reps` times, HIP events around each replay.  Returns {median, p10, p90} in us
    of the per-step mean of each replay."""
    import numpy as np
    stream = torch.cuda.current_stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(chunk):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record(stream)
    for r in range(reps):
        g.replay()
        ev[r + 1].record(stream)
    torch.cuda.synchronize()
    us = np.array([ev[r].elapsed_time(ev[r + 1]) * 1e3 / chunk for r in range(reps)])
    return {"median": round(float(np.median(us)), 3), "p10": round(float(np.percentile(us, 10)), 3),
            "p90": round(float(np.percentile(us, 90)), 3), "replays": reps, "steps_per_replay": chunk}


# --------------------------------------------------------------------- workloads

def bench_expert(torch, steps, warmup, dev):
    from k3hip.moe import expert_ffn_fused
    gen = torch.Generator(device=dev)
    gen.manual_seed(1002)
    experts = [(rand_mxfp4(torch, gen, I, H, dev), rand_mxfp4(torch, gen, I, H, dev),
                rand_mxfp4(torch, gen, H, I, dev)) for _ in range(ROTATE)]
    x = torch.randn(1, H, device=dev, generator=gen).to(torch.bfloat16)
    outs = [torch.empty(1, H, device=dev) for _ in range(2)]

    def step(i):
        outs[i & 1] = expert_ffn_fused(x, *experts[i % ROTATE])

    sec, wall = graph_time(torch, step, steps, warmup)
    stats = None if EAGER else step_stats(torch, step, ROTATE)
    del experts
    return sec, wall, stats


def bench_expert_sustained(torch, steps, dev, reps=8):
    """Independent experts back to back: expert i runs on stream i % 2, so one expert's
    gate/up launch overlaps the other's down GEMV (no dependency between experts, as in a
    layer's top-k).  The graph of `steps` experts is replayed `reps` times; returns seconds
    per expert."""
    from k3hip.moe import expert_ffn_fused
    gen = torch.Generator(device=dev)
    gen.manual_seed(1002)
    experts = [(rand_mxfp4(torch, gen, I, H, dev), rand_mxfp4(torch, gen, I, H, dev),
                rand_mxfp4(torch, gen, H, I, dev)) for _ in range(ROTATE)]
    x = torch.randn(1, H, device=dev, generator=gen).to(torch.bfloat16)
    main = torch.cuda.current_stream()
    side = [torch.cuda.Stream(device=dev) for _ in range(2)]
    outs = [None, None]

    def run(n):
        cur = torch.cuda.current_stream()   # the capture stream inside torch.cuda.graph
        for s in side:
            s.wait_stream(cur)
        for i in range(n):
            with torch.cuda.stream(side[i & 1]):
                outs[i & 1] = expert_ffn_fused(x, *experts[i % ROTATE])
        for s in side:
            cur.wait_stream(s)

    run(4)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(steps)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(main)
    for _ in range(reps):
        g.replay()
    e1.record(main)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / (reps * steps)
    del g, experts
    return sec


def bench_gemv(torch, steps, warmup, dev):
    from k3hip.mxfp4_matvec import mxfp4_matvec_fused
    gen = torch.Generator(device=dev)
    gen.manual_seed(1001)
    ws = [rand_mxfp4(torch, gen, I, H, dev) for _ in range(ROTATE)]
    x = torch.randn(1, H, device=dev, generator=gen).to(torch.bfloat16)

    def step(i):
        mxfp4_matvec_fused(x, *ws[i % ROTATE], out_dtype=torch.bfloat16)

    sec, _ = graph_time(torch, step, steps, warmup)
    return sec, None if EAGER else step_stats(torch, step, ROTATE)


_EXPERTS = []


def resident_experts(torch, dev):
    """384 distinct MXFP4 experts (8.98 GB), built once and shared by the layer and
    prefill workloads."""
    if not _EXPERTS:
        gen = torch.Generator(device=dev)
        gen.manual_seed(1003)
        _EXPERTS.extend((rand_mxfp4(torch, gen, I, H, dev), rand_mxfp4(torch, gen, I, H, dev),
                         rand_mxfp4(torch, gen, H, I, dev)) for _ in range(E_LAYER))
    return _EXPERTS


def build_layer(torch, dev):
    from k3hip.moe import MoEConfig, RoutedMoE
    gen = torch.Generator(device=dev)
    gen.manual_seed(1003)
    experts = resident_experts(torch, dev)
    w = {"gate.weight": (torch.randn(E_LAYER, H, device=dev, generator=gen) * 0.02).to(torch.bfloat16)}
    for name, shape in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        w[f"shared_experts.{name}_proj.weight"] = (torch.randn(*shape, device=dev, generator=gen) * 0.02
                                                   ).to(torch.bfloat16)
    which = {"w1": 0, "w3": 1, "w2": 2}
    cfg = MoEConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E_LAYER, num_experts_per_token=TOPK,
                    shared_intermediate_size=I, router="softmax", activation="silu")
    return RoutedMoE(cfg, 0, w, lambda L, e, wh: experts[e][which[wh]]), experts


def bench_layer(torch, steps, warmup, dev):
    moe, experts = build_layer(torch, dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    xs = torch.randn(steps + warmup + 3, H, device=dev, generator=gen).to(torch.bfloat16)
    touched = set()

    def step(i):
        moe(xs[i:i + 1])

    sec, _ = graph_time(torch, step, steps, warmup)
    stats = None if EAGER else step_stats(torch, step, min(64, steps))
    # distinct experts the timed tokens routed to (evidence the MALL could not hold them)
    for i in range(min(steps, 32)):
        touched.update(moe.route(xs[i:i + 1]).expert_indices.view(-1).tolist())
    del moe
    return sec, len(touched), stats


MULTI_T = 4                     # decode tokens per step of the multi-token layer workload


def bench_layer_multi(torch, steps, warmup, dev, T=MULTI_T):
    """The 384-expert layer for T decode tokens per step (RoutedMoE.__call__ on
    k3_moe_layer_decode_multi: router and shared gate/up rows, top-k, the routed experts over
    the union of the tokens' choices, shared down rows).  Returns seconds for `steps` steps
    and the mean union size / bytes per step, the algorithmic bytes when every union expert,
    the router and the shared expert are read once."""
    import numpy as np
    moe, _ = build_layer(torch, dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(8)
    n = steps + warmup + 3
    xs = torch.randn(n * T, H, device=dev, generator=gen).to(torch.bfloat16)

    def step(i):
        moe(xs[i * T:(i + 1) * T])

    sec, _ = graph_time(torch, step, steps, warmup)
    stats = None if EAGER else step_stats(torch, step, min(64, steps))
    unions = [len(set(moe.route(xs[i * T:(i + 1) * T]).expert_indices.view(-1).tolist())) for i in range(steps)]
    del moe
    u = float(np.mean(unions))
    nbytes = E_LAYER * H * 2 + u * EXPERT_BYTES + 3 * H * I * 2
    return sec, u, nbytes, stats


K3_H, K3_L, K3_I, K3_E, K3_K, K3_IS = 7168, 3584, 3072, 896, 16, 6144
K3_LAYER_BYTES = (K3_E * K3_H * 2 + 2 * K3_L * K3_H * 2 + K3_K * 3 * proj_bytes(K3_I, K3_L)
                  + 3 * K3_IS * K3_H * 2)                                 # 660,602,880
K3_PF_T = 2048
K3_PREFILL = True
K3_MULTI = True


def bench_k3_layer(torch, steps, warmup, dev):
    """K3's routed layer at batch 1 with its latent wrapper (LatentMoE): sigmoid + bias
    routing of x over 896 experts (top-16, renormalised, scaling 2.5), latent down projection
    [3584, 7168] bf16, 16 routed SiTU experts [3072 x 3584] MXFP4 on the latent state, RMS
    norm, up projection [7168, 3584] bf16, two shared experts (one bf16 MLP of width 6144)
    on x.  All 896 experts are distinct and resident (15.7 GB); a fresh token per step."""
    from types import SimpleNamespace
    from k3hip.moe import LatentMoE
    gen = torch.Generator(device=dev)
    gen.manual_seed(1006)
    bf = torch.bfloat16
    experts = [(rand_mxfp4(torch, gen, K3_I, K3_L, dev), rand_mxfp4(torch, gen, K3_I, K3_L, dev),
                rand_mxfp4(torch, gen, K3_L, K3_I, dev)) for _ in range(K3_E)]
    rn = lambda *s: torch.randn(*s, device=dev, generator=gen)  # noqa: E731
    w = {"gate.weight": (rn(K3_E, K3_H) * 0.02).to(bf), "gate.e_score_correction_bias": rn(K3_E) * 0.05,
         "routed_expert_down_proj.weight": (rn(K3_L, K3_H) * 0.02).to(bf),
         "routed_expert_up_proj.weight": (rn(K3_H, K3_L) * 0.02).to(bf),
         "routed_expert_norm.weight": 1.0 + 0.1 * rn(K3_L),
         "shared_experts.gate_proj.weight": (rn(K3_IS, K3_H) * 0.02).to(bf),
         "shared_experts.up_proj.weight": (rn(K3_IS, K3_H) * 0.02).to(bf),
         "shared_experts.down_proj.weight": (rn(K3_H, K3_IS) * 0.02).to(bf)}
    cfg = SimpleNamespace(hidden_size=K3_H, routed_expert_hidden_size=K3_L, moe_intermediate_size=K3_I,
                          num_experts=K3_E, num_experts_per_token=K3_K, moe_renormalize=True,
                          routed_scaling_factor=2.5, situ_beta=2.0, situ_linear_beta=3.0, rms_norm_eps=1e-5)
    which = {"w1": 0, "w3": 1, "w2": 2}
    moe = LatentMoE(cfg, 0, w, lambda L, e, wh: experts[e][which[wh]])
    xs = rn(steps + warmup + 3, K3_H).to(bf)

    def step(i):
        moe(xs[i:i + 1])

    sec, _ = graph_time(torch, step, steps, warmup)
    stats = None if EAGER else step_stats(torch, step, min(64, steps))
    touched = set()
    for i in range(min(steps, 32)):
        touched.update(moe.route(xs[i:i + 1]).expert_indices.view(-1).tolist())
    multi = None
    if K3_MULTI:
        # four decode tokens per step through k3_moe_latent_layer_decode_multi (each expert
        # any of them selects read once), against four single-token steps
        import numpy as np
        ms = min(steps, 64)
        x4 = rn((ms + warmup + 3) * MULTI_T, K3_H).to(bf)

        def mstep(i):
            moe(x4[i * MULTI_T:(i + 1) * MULTI_T])

        msec, _ = graph_time(torch, mstep, ms, min(warmup, 8))
        unions = [len(set(moe.route(x4[i * MULTI_T:(i + 1) * MULTI_T]).expert_indices.view(-1).tolist()))
                  for i in range(ms)]
        u = float(np.mean(unions))
        mbytes = (K3_E * K3_H * 2 + 2 * K3_L * K3_H * 2 + u * 3 * proj_bytes(K3_I, K3_L) + 3 * K3_IS * K3_H * 2)
        mus = msec / ms * 1e6
        multi = {"tokens_per_step": MULTI_T, "us_per_step": round(mus, 2), "us_per_token": round(mus / MULTI_T, 2),
                 "union_experts_mean": round(u, 2), "bytes_per_step_mean": int(mbytes),
                 "GB/s": round(mbytes / (mus * 1e-6) / 1e9, 1),
                 "pct_hbm_peak": round(100 * mbytes / (mus * 1e-6) / 1e9 / HBM_PEAK_GBS, 1),
                 "vs_4_single_token_steps": round(MULTI_T * sec / steps * 1e6 / mus, 3),
                 "what": "LatentMoE.__call__ on 4 tokens: k3_moe_latent_layer_decode_multi (router, latent "
                         "down, shared and up rows for T tokens in HIP; each selected expert read once)"}
        del x4
    prefill = None
    if K3_PREFILL:
        # K3 prefill: 2048 tokens through the same layer, routing included (one router GEMM
        # plus one top-k launch), the experts grouped on the device; no host sync inside
        xp = rn(K3_PF_T, K3_H).to(bf)
        r = moe.route(xp)
        counts = torch.bincount(r.expert_indices.view(-1), minlength=K3_E)
        used = int((counts > 0).sum())

        def pstep(i):
            moe(xp)

        psec, _ = graph_time(torch, pstep, 4, 1)
        pbytes = (used * 3 * proj_bytes(K3_I, K3_L) + K3_E * K3_H * 2 + 2 * K3_L * K3_H * 2
                  + 3 * K3_IS * K3_H * 2 + K3_PF_T * K3_H * (2 + 4))
        pflops = 2 * K3_PF_T * (K3_K * 3 * K3_I * K3_L + K3_E * K3_H + 2 * K3_L * K3_H + 3 * K3_IS * K3_H)
        prefill = {"tokens": K3_PF_T, "ms": round(psec / 4 * 1e3, 3),
                   "tokens_per_s": round(K3_PF_T / (psec / 4), 1),
                   "GB/s": round(pbytes / (psec / 4) / 1e9, 1), "bytes": pbytes,
                   "useful_TFLOP/s": round(pflops / (psec / 4) / 1e12, 1),
                   "experts_used": used, "expert_load_max": int(counts.max()),
                   "what": "LatentMoE.__call__ on 2048 tokens: router GEMM + k3_moe_topk, latent down "
                           "GEMM, k3_moe_grouped_ffn, RMSNorm, up GEMM, shared-expert GEMMs"}
        del xp
    del moe, experts, w
    return sec, len(touched), stats, prefill, multi


def bench_ingest(torch, dev, n_experts=32):
    """Checkpoint ingestion: n K3-shaped experts ([3072 x 3584] MXFP4, three projections,
    reference tensor names) written as one safetensors shard to a temporary directory, then
    made resident through TensorSource.load_experts (one read per adjacent (packed, scale)
    pair into page-locked staging, asynchronous host-to-device copies, device scale check).
    The file is in the page cache, so this is the host-memory -> HBM ingest rate, not SSD."""
    import shutil
    import tempfile
    import numpy as np
    from k3hip.checkpoint import TensorSource, expert_name, write_safetensors
    rng = np.random.default_rng(1007)
    tmp = Path(tempfile.mkdtemp(prefix="k3ingest"))
    try:
        t = {}
        for e in range(n_experts):
            for w, (n, k) in (("w1", (K3_I, K3_L)), ("w3", (K3_I, K3_L)), ("w2", (K3_L, K3_I))):
                t[expert_name(0, e, w) + ".weight_packed"] = (rng.integers(0, 256, (n, k // 2), dtype=np.uint8), "U8")
                t[expert_name(0, e, w) + ".weight_scale"] = (rng.integers(118, 131, (n, k // 32), dtype=np.uint8), "U8")
        write_safetensors(tmp / "model-00001-of-00001.safetensors", t)
        nbytes = sum(a.nbytes for a, _ in t.values())
        del t
        best = None
        for _ in range(3):
            src = TensorSource(ckpt=tmp, device=dev)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            res = src.load_experts(0, n_experts)
            torch.cuda.synchronize()
            dt = time.perf_counter() - t0
            best = dt if best is None else min(best, dt)
            reads = src.reads
            src.close()
            del res
        return {"GB/s": round(nbytes / best / 1e9, 2), "bytes": nbytes, "s": round(best, 4),
                "experts": n_experts, "file_reads": reads, "projections": 3 * n_experts,
                "source": "page cache (a file written just before)"}
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


PF_T, PF_K = 2048, 8
PF_FLOPS = 2 * PF_T * PF_K * 3 * H * I                                   # 1.443e12 useful


def zipf_routing(T, E, k, s=1.1, seed=1004):
    """k distinct experts per token, drawn without replacement with probability ~ r^-s over a
    seeded permutation of the experts (Gumbel top-k); combine weights softmax(N(0,1))."""
    import numpy as np
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    logw = -s * np.log(np.arange(1, E + 1, dtype=np.float64))[np.argsort(perm)]
    g = logw[None, :] - np.log(-np.log(rng.random((T, E))))
    idx = np.argsort(-g, axis=1)[:, :k].astype(np.int32)
    z = rng.standard_normal((T, k))
    w = np.exp(z - z.max(axis=1, keepdims=True))
    return idx, (w / w.sum(axis=1, keepdims=True)).astype(np.float32)


def bench_prefill(torch, steps, warmup, dev):
    """Grouped MoE prefill: 2048 bf16 tokens (hidden 7168), top-8 over the 384 resident
    MXFP4 experts with Zipf(1.1) load; one step = the whole batch through the grouping
    pass, both grouped GEMMs and the combine."""
    import numpy as np
    from k3hip.moe import moe_grouped_ffn
    experts = resident_experts(torch, dev)
    table = torch.tensor([[t.data_ptr() for pair in ex for t in pair] for ex in experts], dtype=torch.int64,
                         device=dev)
    idx_np, w_np = zipf_routing(PF_T, E_LAYER, PF_K)
    idx = torch.from_numpy(idx_np).to(dev)
    w = torch.from_numpy(w_np).to(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1004)
    x = torch.randn(PF_T, H, device=dev, generator=gen).to(torch.bfloat16)

    def step(i):
        moe_grouped_ffn(x, idx, w, table, I, validate=False)

    sec, _ = graph_time(torch, step, steps, warmup)
    counts = np.bincount(idx_np.ravel(), minlength=E_LAYER)
    used = int((counts > 0).sum())
    bytes_ = used * EXPERT_BYTES + PF_T * H * 2 + PF_T * H * 4
    return sec / steps, bytes_, counts


MLA_H, MLA_T = 64, 32768
MLA_BYTES = MLA_T * (512 + 64) * 2 + 2 * MLA_H * 128 * 512 * 2 + MLA_H * 192 * 2 + MLA_H * 128 * 4  # 54,583,296
MLA_F32_BYTES = MLA_BYTES + MLA_T * (512 + 64) * 2                                                  # 92,332,032


def bench_mla(torch, steps, warmup, dev, cache_dtype=None):
    """Latent-MLA absorbed decode: 64 heads over a 32768-token latent cache (kv_lora_rank
    512 + rope 64; bf16, or fp32 as the reference's default cache), W_UK / W_UV
    [64, 128, 512] bf16, scale 1/sqrt(192).  16 distinct caches and 8 weight sets rotate
    (737 MB in bf16) so the MALL cannot hold them."""
    from k3hip.mla import mla_decode_absorbed
    gen = torch.Generator(device=dev)
    gen.manual_seed(1005)
    bf = torch.bfloat16
    cdt = cache_dtype or bf
    caches = [(torch.randn(MLA_T, 512, device=dev, generator=gen).to(cdt),
               torch.randn(MLA_T, 64, device=dev, generator=gen).to(cdt)) for _ in range(16)]
    weights = [((torch.randn(MLA_H, 128, 512, device=dev, generator=gen) * 0.02).to(bf),
                (torch.randn(MLA_H, 128, 512, device=dev, generator=gen) * 0.02).to(bf)) for _ in range(8)]
    q_nope = torch.randn(MLA_H, 128, device=dev, generator=gen).to(bf)
    q_rot = torch.randn(MLA_H, 64, device=dev, generator=gen).to(bf)
    scale = 192 ** -0.5

    def step(i):
        wk, wv = weights[i % 8]
        lat, rot = caches[i % 16]
        mla_decode_absorbed(q_nope, q_rot, wk, wv, lat, rot, scale)

    sec, _ = graph_time(torch, step, steps, warmup)
    stats = None if EAGER else step_stats(torch, step, 32)
    del caches, weights
    return sec, stats


MS_HID, MS_QL = 7168, 1536
MS_BYTES = (2 * (MS_QL * MS_HID + (512 + 64) * MS_HID + MLA_H * 128 * MS_HID + MLA_H * 192 * MS_QL
                 + MS_HID * MLA_H * 128) + MLA_BYTES)                     # 357,490,688


def bench_mla_step(torch, steps, warmup, dev):
    """One decode token through a whole MLA layer at K3 shapes (k3_mla_step_decode): hidden
    7168, q_lora_rank 1536, 64 heads (nope 128, rope 64, v 128), kv_lora_rank 512, output
    gate, bf16 weights, the new cache row written at position 32767 of a bf16 cache.  Two
    weight sets and four caches rotate (1.6 GB), so the MALL cannot hold them."""
    from types import SimpleNamespace
    from k3hip.mla import MLACache, MLAAttention
    cfg = SimpleNamespace(hidden_size=MS_HID, num_attention_heads=MLA_H, q_lora_rank=MS_QL, kv_lora_rank=512,
                          qk_nope_head_dim=128, qk_rope_head_dim=64, v_head_dim=128, q_head_dim=192,
                          rms_norm_eps=1e-5, mla_use_output_gate=True)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1008)
    bf = torch.bfloat16

    def lin(o, i):
        return (torch.randn(o, i, device=dev, generator=gen) / i ** 0.5).to(bf)

    mods = []
    for _ in range(2):
        w = {"q_a_proj.weight": lin(MS_QL, MS_HID), "q_a_layernorm.weight": torch.ones(MS_QL, device=dev),
             "q_b_proj.weight": lin(MLA_H * 192, MS_QL), "kv_a_proj_with_mqa.weight": lin(576, MS_HID),
             "kv_a_layernorm.weight": torch.ones(512, device=dev), "kv_b_proj.weight": lin(MLA_H * 256, 512),
             "g_proj.weight": lin(MLA_H * 128, MS_HID), "o_proj.weight": lin(MS_HID, MLA_H * 128)}
        mods.append(MLAAttention(cfg, w))
    pos = MLA_T - 1
    caches = [MLACache(torch.randn(1, MLA_T, 512, device=dev, generator=gen).to(bf),
                       torch.randn(1, MLA_T, 64, device=dev, generator=gen).to(bf), pos) for _ in range(4)]
    xs = torch.randn(8, 1, 1, MS_HID, device=dev, generator=gen).to(bf)

    def step(i):
        c = caches[i % 4]
        c.length = pos
        mods[i % 2].decode_step(xs[i % 8], c)

    sec, _ = graph_time(torch, step, steps, warmup)
    stats = None if EAGER else step_stats(torch, step, 32)
    del mods, caches
    return sec, stats


KDA_H, KDA_D = 96, 128
KDA_BYTES = 2 * KDA_H * KDA_D * KDA_D * 4 + KDA_H * KDA_D * 4 * 5 + KDA_H * 4   # 12,829,056


def bench_kda(torch, steps, warmup, dev):
    """One KDA recurrent decode step (k3_kda_recurrent_decode) at K3 shapes: 96 heads,
    128 x 128 fp32 state per head (6 MiB, read and written in place), fp32 q/k/v/g/beta.
    32 states rotate (403 MB), so the MALL cannot hold them."""
    import ctypes
    from k3hip import _lib
    gen = torch.Generator(device=dev)
    gen.manual_seed(1009)
    states = [torch.randn(KDA_H, KDA_D, KDA_D, device=dev, generator=gen) * 0.1 for _ in range(32)]
    q, k, v = (torch.nn.functional.normalize(torch.randn(KDA_H, KDA_D, device=dev, generator=gen), dim=-1)
               for _ in range(3))
    g = -5.0 * torch.sigmoid(torch.randn(KDA_H, KDA_D, device=dev, generator=gen))
    beta = torch.sigmoid(torch.randn(KDA_H, device=dev, generator=gen))
    out = torch.empty(KDA_H, KDA_D, device=dev)

    def step(i):
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.call("k3_kda_recurrent_decode", q.data_ptr(), k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(),
                  _lib.K3_F32, states[i % 32].data_ptr(), out.data_ptr(), _lib.K3_F32, KDA_H, KDA_H, KDA_D, KDA_D,
                  KDA_D ** -0.5, st)

    sec, _ = graph_time(torch, step, steps, warmup)
    stats = None if EAGER else step_stats(torch, step, 32)
    # a 256-token prefill through the same recurrence in one launch (k3_kda_recurrent)
    Tp = 256
    qp, kp, vp = (torch.nn.functional.normalize(torch.randn(Tp, KDA_H, KDA_D, device=dev, generator=gen), dim=-1)
                  for _ in range(3))
    gp = -5.0 * torch.sigmoid(torch.randn(Tp, KDA_H, KDA_D, device=dev, generator=gen))
    bp = torch.sigmoid(torch.randn(Tp, KDA_H, device=dev, generator=gen))
    op = torch.empty(Tp, KDA_H, KDA_D, device=dev)

    def prefill(i):
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.call("k3_kda_recurrent", qp.data_ptr(), kp.data_ptr(), vp.data_ptr(), gp.data_ptr(), bp.data_ptr(),
                  _lib.K3_F32, states[i % 32].data_ptr(), op.data_ptr(), _lib.K3_F32, Tp, KDA_H, KDA_H, KDA_D, KDA_D,
                  KDA_D ** -0.5, st)

    psec, _ = graph_time(torch, prefill, 16, 2)
    del states
    return sec, stats, psec / 16, Tp


KS_HID, KS_P = 7168, KDA_H * KDA_D
KS_BYTES = (2 * (5 * KS_P * KS_HID + KDA_D * KS_HID + KS_P * KDA_D + KDA_H * KS_HID)
            + 2 * KDA_H * KDA_D * KDA_D * 4 + 2 * 3 * 3 * KS_P * 4)      # 900,628,480


def bench_kda_step(torch, steps, warmup, dev):
    """One token through a whole KDA layer at K3 shapes (k3_kda_step_decode): hidden 7168,
    96 heads of 128, short convolutions of 4, bf16 projections (887 MB, beyond the MALL),
    fp32 state updated in place, a fresh x per step."""
    from types import SimpleNamespace
    from k3hip.kda import KDAAttention
    cfg = SimpleNamespace(hidden_size=KS_HID, kda_num_heads=KDA_H, kda_head_dim=KDA_D, kda_conv_size=4,
                          kda_gate_lower_bound=-5.0, rms_norm_eps=1e-5)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1010)

    def W(*shape, s=0.02):
        return torch.randn(*shape, device=dev, generator=gen) * s

    a = torch.zeros(KDA_D, device=dev)
    a[:KDA_H] = torch.log(1 + 15 * torch.rand(KDA_H, device=dev, generator=gen))
    w = {"q_proj.weight": W(KS_P, KS_HID), "k_proj.weight": W(KS_P, KS_HID), "v_proj.weight": W(KS_P, KS_HID),
         "g_proj.weight": W(KS_P, KS_HID), "o_proj.weight": W(KS_HID, KS_P),
         "q_conv1d.weight": W(KS_P, 1, 4, s=0.3), "k_conv1d.weight": W(KS_P, 1, 4, s=0.3),
         "v_conv1d.weight": W(KS_P, 1, 4, s=0.3), "f_a_proj.weight": W(KDA_D, KS_HID),
         "f_b_proj.weight": W(KS_P, KDA_D), "b_proj.weight": W(KDA_H, KS_HID), "o_norm.weight": 1 + W(KDA_D, s=0.1),
         "A_log": a, "dt_bias": W(KS_P, s=1.0)}
    attn = KDAAttention(cfg, w)
    del w
    state = torch.randn(KDA_H, KDA_D, KDA_D, device=dev, generator=gen) * 0.1
    conv = [torch.zeros(3, 3, KS_P, device=dev) for _ in range(2)]
    xs = torch.randn(16, KS_HID, device=dev, generator=gen).to(torch.bfloat16)
    out = torch.empty(KS_HID, device=dev)

    def step(i):
        attn.decode_step(xs[i % 16], state, conv[i % 2], conv[(i + 1) % 2], out)

    sec, _ = graph_time(torch, step, steps, warmup)
    stats = None if EAGER else step_stats(torch, step, 32)
    # a 256-token prompt through KDAAttention's prefill path (eager: GEMMs on the BLAS
    # library, one recurrence launch), timed with events
    xp = torch.randn(1, 256, KS_HID, device=dev, generator=gen).to(torch.bfloat16)
    attn(xp)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        attn(xp)
    e1.record()
    torch.cuda.synchronize()
    pre = e0.elapsed_time(e1) / 3 / 1e3
    del attn
    return sec, stats, pre


def bench_read_ceiling(torch, nbytes, steps, dev):
    """One streaming-read launch of nbytes (the library's calibration kernel), rotating
    over >= 1.5 GB of buffers: the bandwidth a single launch of this size can reach."""
    import ctypes
    from k3hip import _lib
    nbuf = max(4, min(64, -(-(3 << 29) // nbytes)))
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(nbuf)]
    sink = torch.empty(4096, dtype=torch.uint8, device=dev)

    def step(i):
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.call("k3_stream_read", ctypes.c_void_p(bufs[i % nbuf].data_ptr()), nbytes,
                  ctypes.c_void_p(sink.data_ptr()), st)

    sec, _ = graph_time(torch, step, steps, 8)
    del bufs
    return sec / steps


def bench_copy_ceiling(torch, nbytes, steps, dev):
    """One streaming-copy launch of nbytes (k3_stream_copy) rotating over 16 source /
    destination pairs: the known-size kernel the profiler's WRITE_SIZE counter is scaled by."""
    import ctypes
    from k3hip import _lib
    src = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(16)]
    dst = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(16)]

    def step(i):
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.call("k3_stream_copy", ctypes.c_void_p(dst[i % 16].data_ptr()),
                  ctypes.c_void_p(src[i % 16].data_ptr()), nbytes, st)

    sec, _ = graph_time(torch, step, steps, 8)
    del src, dst
    return sec / steps


def bench_cpu(sample_s=12.0):
    """torch-CPU restatement of the k3ref expert path (k3ref/layers.py:226-234 with the
    decode of k3ref/weights.py:29-37 on every access), timed on this host."""
    import numpy as np
    import torch

    from oracle import cpu_baseline
    n = len(os.sched_getaffinity(0))
    torch.set_num_threads(n)
    out = cpu_baseline.time_expert(H, I, sample_s=sample_s, threads=n)
    one = cpu_baseline.time_expert(H, I, sample_s=sample_s / 4, threads=1)
    out["single_thread"] = {k: one[k] for k in ("value", "unit", "cores", "ms_per_expert", "matmul_only_GB/s",
                                                "matmul_only_ms", "sample")}
    out["projection"] = cpu_baseline.time_projection(I, H, sample_s=sample_s / 6, threads=n)
    out["projection_single_thread"] = cpu_baseline.time_projection(I, H, sample_s=sample_s / 6, threads=1)
    torch.set_num_threads(n)
    out["moe_layer"] = cpu_baseline.time_layer(H, I, E_LAYER, TOPK, sample_s=sample_s / 2, threads=n)
    out["mla_decode"] = cpu_baseline.time_mla(MLA_H, MLA_T, sample_s=sample_s / 3, threads=n)
    return out


def kernel_sources_sha256():
    """sha256 over the kernel sources (csrc/*.hip, *.h, in name order): the identity of the
    kernels a counter record was measured on."""
    import hashlib
    h = hashlib.sha256()
    for f in sorted((ROOT / "kimi-k3-mlx-macmini_amd" / "csrc").glob("*")):
        if f.suffix in (".hip", ".h"):
            h.update(f.name.encode())
            h.update(f.read_bytes())
    return h.hexdigest()


COUNTERS_CURRENT = None   # set by counters_from_profiles: the record matches today's kernel sources


def counters_from_profiles():
    """Per-workload counter figures (rocprofv3 FETCH_SIZE / WRITE_SIZE / MFMA counts over the
    same workloads, calibrated bytes, kernel times) from the committed profiles/counters.json,
    with whether its kernel-source hash matches the sources of this run (the fields say
    "stale" when it does not)."""
    global COUNTERS_CURRENT
    f = ROOT / "profiles" / "counters.json"
    try:
        d = json.loads(f.read_text())
    except (ValueError, OSError):
        return {}
    COUNTERS_CURRENT = d.get("csrc_sha256") == kernel_sources_sha256()
    return d.get("workloads", {})


def counter_fields(rec):
    """`traffic` (counter bytes / algorithmic bytes per step) and, for the MFMA workloads,
    `mfma_util`, from one profiles/counters.json record."""
    if not rec:
        return {}
    src = "profiles/counters.json" + ("" if COUNTERS_CURRENT else " (stale: measured on other kernel sources)")
    out = {"traffic": {"ratio": rec["traffic_ratio"], "counter_bytes": rec["counter_bytes"],
                       "algorithmic_bytes": rec["algorithmic_bytes"], "source": src,
                       "current": bool(COUNTERS_CURRENT)},
           # each launch's mean kernel time (eager, under the profiler) and the HBM bytes its
           # counters show, so the throughput of each launch stands beside the step's
           "launches": [{"kernel": k["kernel"], "avg_us": k["avg_us"], "counter_bytes": k["bytes"],
                         "GB/s": round(k["bytes"] / (k["avg_us"] * 1e-6) / 1e9, 1),
                         "pct_hbm_peak": round(100 * k["bytes"] / (k["avg_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 1)}
                        for k in rec.get("kernels", []) if k.get("avg_us")]}
    m = rec.get("mfma")
    if m:
        u = {"mfma": m["type"], "executed_TFLOP/s": m["executed_TFLOP/s"],
             "frac_of_issue_peak": m["executed_frac_of_issue_peak"], "issue_peak_TFLOP/s": m["issue_peak_TFLOP/s"]}
        if "useful_frac_of_mxfp4_peak" in m:
            u["useful_frac_of_mxfp4_peak"] = m["useful_frac_of_mxfp4_peak"]
        u["current"] = bool(COUNTERS_CURRENT)
        out["mfma_util"] = u
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--workloads",
                    default="expert,sustained,layer,layer4,k3layer,ingest,prefill,gemv,mla,mlaf32,mlastep,kda,"
                            "kdastep,ceiling")
    ap.add_argument("--eager", action="store_true",
                    help="launch steps one by one instead of replaying a HIP graph (profiler counter runs)")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: k3hip runs on one GPU only (no multi-GPU path); use --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(2)
    import k3hip
    k3hip.lib()   # fails loudly when libk3hip.so is missing: there is no fallback
    dev = torch.device("cuda:0")
    work = set(args.workloads.split(","))
    K, W = args.steps, args.warmup

    cnt = counters_from_profiles()
    sec, wall, estats = bench_expert(torch, K, W, dev)
    per_step = sec / K
    gbs = EXPERT_BYTES / per_step / 1e9
    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(per_step * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4xbf16->f32",
        "data": "synthetic (seeded random MXFP4 weights, E8M0 in [118,130], bf16 x ~ N(0,1))",
        "config": {"workload": "expert_swiglu_ffn_b1", "hidden": H, "intermediate": I,
                   "experts_rotated": ROTATE, "act": "silu", "x": "bf16", "out": "f32"},
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": cnt.get("expert_swiglu_ffn_b1", {}).get("counter_bytes") if COUNTERS_CURRENT else None,
                     "kernel": "expert FFN step: expert_gateup_kernel then gemv_kernel (down)",
                     "launches_per_step": 2, "bytes_per_step": EXPERT_BYTES,
                     "avg_step_us": round(per_step * 1e6, 3)},
        "wall_s": round(wall, 4),
        "step_us": estats,
    }
    if "sustained" in work:
        ssec_ = bench_expert_sustained(torch, ROTATE, dev)
        sgbs_ = EXPERT_BYTES / ssec_ / 1e9
        line["sustained"] = {"us_per_expert": round(ssec_ * 1e6, 3), "GB/s": round(sgbs_, 1),
                             "pct_hbm_peak": round(100 * sgbs_ / HBM_PEAK_GBS, 1),
                             "what": "independent experts back to back on two streams (expert i on "
                                     "stream i % 2), graph of 64 replayed 8 times"}
    if "layer" in work:
        lsec, touched, lstats = bench_layer(torch, min(K, 256), min(W, 32), dev)
        lus = lsec / min(K, 256) * 1e6
        lgbs = LAYER_BYTES / (lus * 1e-6) / 1e9
        line["moe_layer"] = {"us_per_layer": round(lus, 2), "GB/s": round(lgbs, 1),
                             "pct_hbm_peak": round(100 * lgbs / HBM_PEAK_GBS, 1),
                             "bytes_per_layer": LAYER_BYTES, "experts": E_LAYER, "top_k": TOPK,
                             "shared_expert": "bf16", "distinct_experts_routed_first32": touched,
                             "launches_per_layer": 3, "step_us": lstats,
                             **counter_fields(cnt.get("moe_layer_b1"))}
        # the batch-1 MXFP4 GEMV sustained inside the layer: its routed gate/up launch (the 8
        # selected experts' gate and up rows back to back, with the shared down rows)
        l2 = [x for x in line["moe_layer"].get("launches", []) if x["kernel"].startswith("layer_l2")]
        if l2:
            line["sustained_in_layer"] = {
                "kernel": l2[0]["kernel"], "GB/s": l2[0]["GB/s"], "pct_hbm_peak": l2[0]["pct_hbm_peak"],
                "what": "the 384-expert layer's routed gate/up launch (8 experts' MXFP4 gate/up GEMVs "
                        "and the shared down rows): counter bytes / kernel-trace time",
                "source": line["moe_layer"]["traffic"]["source"], "current": line["moe_layer"]["traffic"]["current"]}
    if "layer4" in work:
        ms4 = min(K, 128)
        msec4, union4, bytes4, mstats4 = bench_layer_multi(torch, ms4, min(W, 16), dev)
        mus4 = msec4 / ms4 * 1e6
        line["moe_layer_t4"] = {
            "us_per_step": round(mus4, 2), "tokens_per_step": MULTI_T, "us_per_token": round(mus4 / MULTI_T, 2),
            "union_experts_mean": round(union4, 2), "bytes_per_step_mean": int(bytes4),
            "GB/s": round(bytes4 / (mus4 * 1e-6) / 1e9, 1),
            "pct_hbm_peak": round(100 * bytes4 / (mus4 * 1e-6) / 1e9 / HBM_PEAK_GBS, 1),
            "bytes_if_per_token": MULTI_T * LAYER_BYTES,
            "what": "RoutedMoE on 4 tokens: k3_moe_layer_decode_multi (router and shared rows on the "
                    "T-token row kernel, top-k, the union of the routed experts each read once)",
            "step_us": mstats4, **counter_fields(cnt.get("moe_layer_t4"))}
        if "moe_layer" in line:
            line["moe_layer_t4"]["vs_4_single_token_layers"] = round(4 * line["moe_layer"]["us_per_layer"] / mus4, 3)
    if "k3layer" in work:
        ks = min(K, 256)
        ksec, ktouched, kstats, kpre, kmulti = bench_k3_layer(torch, ks, min(W, 32), dev)
        kus = ksec / ks * 1e6
        kgbs = K3_LAYER_BYTES / (kus * 1e-6) / 1e9
        line["k3_latent_layer"] = {"us_per_token": round(kus, 2), "GB/s": round(kgbs, 1),
                                   "pct_hbm_peak": round(100 * kgbs / HBM_PEAK_GBS, 1),
                                   "bytes_per_token": K3_LAYER_BYTES, "hidden": K3_H, "latent": K3_L,
                                   "expert_intermediate": K3_I, "experts": K3_E, "top_k": K3_K,
                                   "shared_intermediate": K3_IS, "router": "sigmoid + bias",
                                   "act": "situ", "distinct_experts_routed_first32": ktouched,
                                   "launches_per_token": 4, "step_us": kstats, "prefill": kpre,
                                   "four_tokens": kmulti,
                                   **counter_fields(cnt.get("k3_latent_layer_b1"))}
        if kmulti is not None:
            kmulti.update(counter_fields(cnt.get("k3_latent_layer_t4")))
        if kpre is not None:
            kpre.update({"grouped_experts_" + k_: v_ for k_, v_ in
                         counter_fields(cnt.get("k3_prefill_t2048_e896_grouped")).items()})
    if "ingest" in work:
        line["checkpoint_ingest"] = bench_ingest(torch, dev)
    if "prefill" in work:
        pst, pbytes, counts = bench_prefill(torch, 8, 2, dev)
        line["moe_prefill"] = {
            "ms": round(pst * 1e3, 3), "GB/s": round(pbytes / pst / 1e9, 1),
            "pct_hbm_peak": round(100 * pbytes / pst / 1e9 / HBM_PEAK_GBS, 1), "bytes": pbytes,
            "useful_TFLOP/s": round(PF_FLOPS / pst / 1e12, 1),
            "mfma": "v_mfma_scale_f32_16x16x128_f8f6f4 (MXFP4 x E4M3 terms; issues at the FP8 rate)",
            "pct_fp8_mfma_peak": round(100 * PF_FLOPS / pst / 5.0e15, 1),
            "tokens": PF_T, "top_k": PF_K, "experts": E_LAYER, "routing": "zipf(1.1), seeded",
            "expert_load": {"max": int(counts.max()), "mean": round(float(counts.mean()), 1),
                            "empty": int((counts == 0).sum())},
            **counter_fields(cnt.get("moe_prefill_t2048_e384"))}
    if "mla" in work:
        ms = min(K, 256)
        msec, mstats = bench_mla(torch, ms, min(W, 32), dev)
        mus = msec / ms * 1e6
        mgbs = MLA_BYTES / (mus * 1e-6) / 1e9
        line["mla_decode"] = {"us": round(mus, 2), "GB/s": round(mgbs, 1),
                              "pct_hbm_peak": round(100 * mgbs / HBM_PEAK_GBS, 1), "bytes": MLA_BYTES,
                              "heads": MLA_H, "tokens": MLA_T, "kv_lora_rank": 512, "rope": 64,
                              "cache": "bf16", "launches": 4, "step_us": mstats,
                              **counter_fields(cnt.get("mla_decode_h64_t32768"))}
    if "mlaf32" in work:
        ms = min(K, 128)
        fsec, fstats = bench_mla(torch, ms, min(W, 16), dev, cache_dtype=torch.float32)
        fus = fsec / ms * 1e6
        fgbs = MLA_F32_BYTES / (fus * 1e-6) / 1e9
        line["mla_decode_f32_cache"] = {
            "us": round(fus, 2), "GB/s": round(fgbs, 1), "pct_hbm_peak": round(100 * fgbs / HBM_PEAK_GBS, 1),
            "bytes": MLA_F32_BYTES, "heads": MLA_H, "tokens": MLA_T, "cache": "fp32 (the reference's default)",
            "what": "k3_mla_decode_absorbed_f32: fp32 rows split into hi/lo bf16 planes as staged",
            "launches": 4, "step_us": fstats, **counter_fields(cnt.get("mla_decode_f32_cache_h64_t32768"))}
    if "mlastep" in work:
        ms_ = min(K, 128)
        ssec, sstats = bench_mla_step(torch, ms_, min(W, 16), dev)
        sus = ssec / ms_ * 1e6
        sgbs = MS_BYTES / (sus * 1e-6) / 1e9
        line["mla_step"] = {"us": round(sus, 2), "GB/s": round(sgbs, 1), "pct_hbm_peak": round(100 * sgbs / HBM_PEAK_GBS, 1),
                            "bytes": MS_BYTES, "hidden": MS_HID, "q_lora_rank": MS_QL, "heads": MLA_H,
                            "tokens": MLA_T, "weights": "bf16", "output_gate": True, "launches": 7,
                            "step_us": sstats}
    if "kda" in work:
        ks_ = min(K, 256)
        kdsec, kdstats, kpre, kTp = bench_kda(torch, ks_, min(W, 32), dev)
        kus = kdsec / ks_ * 1e6
        kgb = KDA_BYTES / (kus * 1e-6) / 1e9
        line["kda_decode"] = {"us": round(kus, 3), "GB/s": round(kgb, 1), "pct_hbm_peak": round(100 * kgb / HBM_PEAK_GBS, 1),
                              "bytes": KDA_BYTES, "heads": KDA_H, "key_dim": KDA_D, "value_dim": KDA_D,
                              "state": "fp32, in place", "launches": 1, "step_us": kdstats,
                              "prefill": {"tokens": kTp, "us": round(kpre * 1e6, 1),
                                          "us_per_token": round(kpre * 1e6 / kTp, 3),
                                          "launches": 1, "what": "k3_kda_recurrent, state kept in registers"}}
    if "kdastep" in work:
        kss = min(K, 128)
        ksec, kstats2, kpre2 = bench_kda_step(torch, kss, min(W, 16), dev)
        kus2 = ksec / kss * 1e6
        kgb2 = KS_BYTES / (kus2 * 1e-6) / 1e9
        line["kda_step"] = {"us": round(kus2, 2), "GB/s": round(kgb2, 1), "pct_hbm_peak": round(100 * kgb2 / HBM_PEAK_GBS, 1),
                            "bytes": KS_BYTES, "hidden": KS_HID, "heads": KDA_H, "head_dim": KDA_D, "conv": 4,
                            "weights": "bf16", "launches": 4, "step_us": kstats2,
                            "prefill_256_tokens": {"ms": round(kpre2 * 1e3, 3), "tokens_per_s": round(256 / kpre2, 1),
                                                   "what": "KDAAttention.prefill: BLAS GEMMs + one k3_kda_recurrent"}}
    if "ceiling" in work:
        ce = bench_read_ceiling(torch, EXPERT_BYTES, 256, dev)
        cl = bench_read_ceiling(torch, LAYER_BYTES, 64, dev)
        cc = bench_copy_ceiling(torch, EXPERT_BYTES, 64, dev)
        line["read_ceiling"] = {
            "what": "single streaming-read launch of the same byte count (k3_stream_read)",
            "expert_bytes_us": round(ce * 1e6, 3), "expert_bytes_GB/s": round(EXPERT_BYTES / ce / 1e9, 1),
            "layer_bytes_us": round(cl * 1e6, 2), "layer_bytes_GB/s": round(LAYER_BYTES / cl / 1e9, 1),
            "copy_expert_bytes_us": round(cc * 1e6, 3),
            "copy_expert_bytes_GB/s": round(2 * EXPERT_BYTES / cc / 1e9, 1)}
        line["pct_of_measured_read"] = round(100 * gbs / (EXPERT_BYTES / ce / 1e9), 1)
        if "moe_layer" in line:
            line["moe_layer"]["pct_of_measured_read"] = round(
                100 * line["moe_layer"]["GB/s"] / (LAYER_BYTES / cl / 1e9), 1)
    if "gemv" in work:
        gsec, gstats = bench_gemv(torch, K, W, dev)
        gus = gsec / K * 1e6
        line["gemv"] = {"us": round(gus, 3), "GB/s": round(GEMV_BYTES / (gus * 1e-6) / 1e9, 1),
                        "shape": [I, H], "x": "bf16", "out": "bf16", "bytes": GEMV_BYTES, "step_us": gstats}
        if "ceiling" in work:
            cg = bench_read_ceiling(torch, GEMV_BYTES, 256, dev)
            line["gemv"]["read_ceiling_us"] = round(cg * 1e6, 3)
            line["gemv"]["read_ceiling_GB/s"] = round(GEMV_BYTES / cg / 1e9, 1)
            line["gemv"]["pct_of_measured_read"] = round(100 * cg * 1e6 / gus, 1)
    if not args.no_cpu:
        cpu = bench_cpu(args.cpu_seconds)
        line["cpu_baseline"] = cpu
        line["gpu_vs_cpu"] = round(gbs / cpu["value"], 1) if cpu.get("value") else None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
