"""The C-ABI from several host threads at once.

The reference runs its kernels from one worker thread (air_llm/server/engine.py:275-291); the
library promises more: stateless entry points on the caller's stream, safe from any thread,
with a thread-local error message.  Four threads, each on its own stream (default priority),
run the expert FFN and the MXFP4 matvec repeatedly while another thread keeps making
matvec calls the library rejects (K not a multiple of 32); every result must equal the
single-threaded one bit for bit (the kernels are deterministic), and each rejected call
must report its own error.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

from oracle import mxfp4 as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _dev(pair):
    return tuple(torch.from_numpy(a).to(DEV) for a in pair)


def test_threads_on_their_own_streams_match_one_thread():
    from k3hip.moe import expert_ffn_fused
    from k3hip.mxfp4_matvec import mxfp4_matvec_fused
    rng = np.random.default_rng(77)
    H, I = 2048, 512
    experts = [tuple(_dev(om.random_mxfp4(rng, *shape)) for shape in ((I, H), (I, H), (H, I))) for _ in range(4)]
    xs = [torch.from_numpy(om.bf16_round(rng.standard_normal((1, H)).astype(np.float32))).to(DEV).to(torch.bfloat16)
          for _ in range(4)]
    want_ffn = [expert_ffn_fused(xs[t], *experts[t]).clone() for t in range(4)]
    want_mv = [mxfp4_matvec_fused(xs[t], *experts[t][0]).clone() for t in range(4)]
    torch.cuda.synchronize()

    rounds = 50
    results: dict[int, list] = {}
    errors: list[str] = []
    bad_msgs: list[str] = []
    start = threading.Barrier(5)

    def worker(t):
        try:
            s = torch.cuda.Stream()
            outs = []
            start.wait()
            with torch.cuda.stream(s):
                for _ in range(rounds):
                    outs.append((expert_ffn_fused(xs[t], *experts[t]), mxfp4_matvec_fused(xs[t], *experts[t][0])))
            s.synchronize()
            results[t] = outs
        except Exception as e:  # reported below with the thread's index
            errors.append(f"thread {t}: {e!r}")

    def failing():
        # raw C-ABI calls rejected by the library itself (K not a multiple of 32), a
        # different K each time, so each message must name the K of its own call
        from k3hip import _lib
        from k3hip import _torch as T
        # buffers sized for the largest K passed, so a regression in the library's own
        # validation shows up as a missing error rather than as reads past an allocation
        kmax = H + 16 + 32 * (rounds - 1)
        x0 = torch.zeros((1, kmax), dtype=torch.bfloat16, device=DEV)
        p0 = torch.zeros((I, kmax // 2), dtype=torch.uint8, device=DEV)
        s0 = torch.full((I, -(-kmax // 32)), 127, dtype=torch.uint8, device=DEV)
        out = torch.empty((1, I), dtype=torch.float32, device=DEV)
        start.wait()
        for i in range(rounds):
            K = H + 16 + 32 * i
            try:
                _lib.call("k3_mxfp4_matvec", T.ptr(x0), _lib.K3_BF16, T.ptr(p0), T.ptr(s0), T.ptr(out), _lib.K3_F32,
                          1, I, K, T.stream(x0))
                bad_msgs.append((K, "no error"))
            except ValueError as e:
                bad_msgs.append((K, str(e)))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)] + [threading.Thread(target=failing)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a thread did not finish"
    assert not errors, errors
    for t in range(4):
        assert len(results[t]) == rounds
        for ffn, mv in results[t]:
            assert torch.equal(ffn, want_ffn[t]) and torch.equal(mv, want_mv[t])
    # every rejected call raised, with the message of its own call
    assert len(bad_msgs) == rounds and all(f"K={K} " in m for K, m in bad_msgs), bad_msgs[:3]


def test_moe_layer_from_threads_matches_one_thread():
    """Three threads decode tokens through one RoutedMoE on their own streams: each stream
    gets its own workspace (arrival counters included), so the launches of different
    threads never meet, and every output equals the same token's output on one thread."""
    from k3hip.moe import RoutedMoE
    from test_gpu_moe_layer import make_layer
    cfg, w, source, *_ = make_layer(5, 1024, 256, 64, 8, 512)
    moe = RoutedMoE(cfg, 0, w, source)
    rng = np.random.default_rng(6)
    xs = [torch.from_numpy(om.bf16_round(rng.standard_normal((1, 1024)).astype(np.float32))).to(DEV).to(torch.bfloat16)
          for _ in range(3)]
    want = [moe(x).clone() for x in xs]
    torch.cuda.synchronize()
    rounds = 40
    results: dict[int, list] = {}
    errors: list[str] = []
    start = threading.Barrier(3)

    def worker(t):
        try:
            s = torch.cuda.Stream()
            start.wait()
            with torch.cuda.stream(s):
                outs = [moe(xs[t]) for _ in range(rounds)]
            s.synchronize()
            results[t] = outs
        except Exception as e:  # reported below with the thread's index
            errors.append(f"thread {t}: {e!r}")

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(3)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a thread did not finish"
    assert not errors, errors
    for t in range(3):
        assert len(results[t]) == rounds and all(torch.equal(y, want[t]) for y in results[t])
