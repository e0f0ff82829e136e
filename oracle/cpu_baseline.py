"""CPU baseline for bench.py (test infrastructure only: timed, never shipped).

A torch-CPU restatement of the reference CPU path for one routed expert:
``k3ref.layers.LatentMoE.expert_forward`` (k3ref/layers.py:226-234) with the weights
decoded on every access as ``k3ref.weights.WeightStore.expert`` does
(k3ref/weights.py:117-122 -> decode_mxfp4, k3ref/weights.py:29-37), fp32 matmuls, SwiGLU.
Two timings:

* ``value``      k3ref-faithful: decode (NumPy, as k3ref) + fp32 matmuls per call
* ``matmul_only`` weights pre-decoded to fp32, matmuls only

Both are expressed in the GPU metric's unit (algorithmic MXFP4 bytes per second) so the
line can be read side by side with the GPU number.
"""
from __future__ import annotations

import os
import platform
import subprocess
import time

import numpy as np

from .mxfp4 import bf16_round, decode_mxfp4, random_mxfp4


def _cpu_model() -> str:
    """The host CPU's model name as /proc/cpuinfo and lscpu give it (lscpu's BIOS model name
    added when it says more, e.g. on virtual machines that report a generic family name)."""
    names = []
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    names.append(line.split(":", 1)[1].strip())
                    break
    except OSError:
        pass
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            if key.strip().lower() in ("model name", "bios model name") and val.strip() and val.strip() not in names:
                names.append(val.strip())
    except (OSError, subprocess.SubprocessError):
        pass
    return " / ".join(names) or platform.processor() or "unknown"


def time_expert(H: int, I: int, sample_s: float = 12.0, threads: int | None = None, seed: int = 1002) -> dict:
    import torch

    threads = threads or len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    rng = np.random.default_rng(seed)
    gate, up, down = random_mxfp4(rng, I, H), random_mxfp4(rng, I, H), random_mxfp4(rng, H, I)
    x = torch.from_numpy(bf16_round(rng.standard_normal((1, H)).astype(np.float32)))
    nbytes = sum(p.nbytes + s.nbytes for p, s in (gate, up, down))

    def faithful():
        w1 = torch.from_numpy(decode_mxfp4(*gate))
        w3 = torch.from_numpy(decode_mxfp4(*up))
        g, u = x @ w1.T, x @ w3.T
        act = torch.nn.functional.silu(g) * u
        del w1, w3
        w2 = torch.from_numpy(decode_mxfp4(*down))
        return act @ w2.T

    W = [torch.from_numpy(decode_mxfp4(*p)) for p in (gate, up, down)]

    def matmul_only():
        g, u = x @ W[0].T, x @ W[1].T
        return (torch.nn.functional.silu(g) * u) @ W[2].T

    def run(fn, budget):
        fn()
        times = []
        t_end = time.perf_counter() + budget
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return float(np.median(times)), len(times)

    t_f, n_f = run(faithful, sample_s * 0.75)
    t_m, n_m = run(matmul_only, sample_s * 0.25)
    return {
        "value": round(nbytes / t_f / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{n_f} calls of one {H}x{I} SwiGLU expert (decode on every call as k3ref, fp32 torch "
                   f"matmuls; NumPy decode runs on 1 thread), median {t_f * 1e3:.1f} ms/expert"),
        "ms_per_expert": round(t_f * 1e3, 2),
        "matmul_only_GB/s": round(nbytes / t_m / 1e9, 3),
        "matmul_only_ms": round(t_m * 1e3, 3),
        "cpu": _cpu_model(),
    }


def _run(fn, budget):
    fn()
    times = []
    t_end = time.perf_counter() + budget
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def time_layer(H: int, I: int, E: int, k: int, sample_s: float = 6.0, threads: int | None = None,
               pool: int = 16, seed: int = 1003) -> dict:
    """The 384-expert layer at batch 1 on the CPU (k3ref/layers.py:214-261 with the softmax
    router): router logits, softmax top-k, the k selected experts decoded on access and run
    in fp32, the bf16 shared expert in fp32.  The expert weights come from a pool of
    ``pool`` random experts (index mod pool), so each call decodes k experts as k3ref does
    without 9 GB of host weights."""
    import torch

    threads = threads or len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    rng = np.random.default_rng(seed)
    experts = [(random_mxfp4(rng, I, H), random_mxfp4(rng, I, H), random_mxfp4(rng, H, I)) for _ in range(pool)]
    wr = torch.from_numpy(bf16_round((rng.standard_normal((E, H)) * 0.02).astype(np.float32)))
    sh = [torch.from_numpy(bf16_round((rng.standard_normal(s) * 0.02).astype(np.float32)))
          for s in ((I, H), (I, H), (H, I))]
    xs = [torch.from_numpy(bf16_round(rng.standard_normal((1, H)).astype(np.float32))) for _ in range(8)]
    it = [0]

    def layer():
        x = xs[it[0] % 8]
        it[0] += 1
        p = torch.softmax(x @ wr.T, dim=-1)
        w, idx = torch.topk(p, k, dim=-1)
        y = torch.zeros(1, H)
        for j in range(k):
            g, u, d = experts[int(idx[0, j]) % pool]
            a = torch.nn.functional.silu(x @ torch.from_numpy(decode_mxfp4(*g)).T) * (x @ torch.from_numpy(decode_mxfp4(*u)).T)
            y += w[0, j] * (a @ torch.from_numpy(decode_mxfp4(*d)).T)
        a = torch.nn.functional.silu(x @ sh[0].T) * (x @ sh[1].T)
        return y + a @ sh[2].T

    t, n = _run(layer, sample_s)
    return {"ms": round(t * 1e3, 2), "calls": n, "cores": threads,
            "sample": (f"{n} calls of the {E}-expert top-{k} layer with a bf16 shared expert (softmax router, "
                       f"{k} experts decoded on access from a pool of {pool}, fp32 torch matmuls), median")}


def time_mla(H: int, T: int, sample_s: float = 4.0, threads: int | None = None, seed: int = 1005) -> dict:
    """The absorbed MLA decode core on the CPU as the reference computes it
    (attention_mla.py:85-87, 193-212): the bf16 cache upcast to fp32 every step, fp32
    products and softmax."""
    import torch

    threads = threads or len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    lat = torch.randn(T, 512, generator=g).to(torch.bfloat16)
    rot = torch.randn(T, 64, generator=g).to(torch.bfloat16)
    wk = (torch.randn(H, 128, 512, generator=g) * 0.02).to(torch.bfloat16)
    wv = (torch.randn(H, 128, 512, generator=g) * 0.02).to(torch.bfloat16)
    qn = torch.randn(H, 1, 128, generator=g)
    qr = torch.randn(H, 1, 64, generator=g)

    def core():
        latf, rotf = lat.float(), rot.float()
        qa = qn @ wk.float()                                      # [H, 1, 512]
        s = (qa @ latf.T + qr @ rotf.T) * 192 ** -0.5             # [H, 1, T]
        p = torch.softmax(s, dim=-1)
        return (p @ latf) @ wv.float().transpose(1, 2)            # [H, 1, 128]

    t, n = _run(core, sample_s)
    return {"ms": round(t * 1e3, 2), "calls": n, "cores": threads,
            "sample": f"{n} calls of the absorbed core, {H} heads over {T} bf16 cache rows (fp32 upcast per call), median"}


def time_projection(N: int, K: int, sample_s: float = 3.0, threads: int | None = None, seed: int = 1001) -> dict:
    """One MXFP4 projection y = x W^T (C1), the reference's own one-projection timing
    (tests/test_mxfp4_kernel.py:87-119): decode on every call (k3ref) then one fp32 matvec,
    plus the matvec alone on pre-decoded weights."""
    import torch

    threads = threads or len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    rng = np.random.default_rng(seed)
    packed, scales = random_mxfp4(rng, N, K)
    x = torch.from_numpy(bf16_round(rng.standard_normal((1, K)).astype(np.float32)))
    nbytes = packed.nbytes + scales.nbytes

    def faithful():
        return x @ torch.from_numpy(decode_mxfp4(packed, scales)).T

    Wd = torch.from_numpy(decode_mxfp4(packed, scales))

    def matmul_only():
        return x @ Wd.T

    t_f, n_f = _run(faithful, sample_s * 0.75)
    t_m, n_m = _run(matmul_only, sample_s * 0.25)
    return {"ms": round(t_f * 1e3, 3), "GB/s": round(nbytes / t_f / 1e9, 3), "calls": n_f, "cores": threads,
            "matmul_only_ms": round(t_m * 1e3, 4), "matmul_only_GB/s": round(nbytes / t_m / 1e9, 3),
            "sample": f"{n_f} calls of one [{N} x {K}] projection (decode + fp32 matvec), median"}
