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
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return platform.processor() or "unknown"


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
