"""MoE routing / expert FFN / layer-combine oracle (test infrastructure only).

Follows ``k3ref/layers.py:198-261`` (``LatentMoE``) and ``air_llm/models/kimi_k3/moe.py:65-132``:

* ``route_softmax``     softmax over router logits, top-k, optional renormalisation by
                        ``sum + 1e-20`` and a scaling factor (the reference's weight
                        convention, ``k3ref/layers.py:221-224``).
* ``route_sigmoid_bias`` the reference router: sigmoid scores, selection on
                        ``scores + bias``, weights gathered from the RAW scores
                        (``k3ref/layers.py:214-224``, ``moe.py:65-76``).
* ``expert_ffn``        ``act(x Wg^T, x Wu^T) Wd^T`` with ``act`` = SwiGLU
                        (``silu(g) * u``, ``ops.py:42-43``) or SiTU (``ops.py:17-28``,
                        ``k3ref/layers.py:53-60``).
* ``moe_layer``         weighted sum of the routed experts plus the shared expert on the
                        original hidden state (``k3ref/layers.py:241-261``).
* ``latent_moe``        K3's layer (``moe.py:110-132``): route on the hidden state, project
                        it to the latent width (``routed_expert_down_proj``), run the routed
                        experts there, RMS-normalise their weighted sum
                        (``routed_expert_norm``, ``ops.py:11-14``), project back to the hidden
                        width (``routed_expert_up_proj``) and add the shared expert applied to
                        the original hidden state.

Everything is float64.  Ties in top-k go to the lower expert index.

Pinning (``tests/test_oracle_moe.py``): softmax/top-k against ``torch.softmax`` /
``torch.topk`` as library routines plus the invariants of ``tests/test_k3ref_layers.py:113-127``
(k distinct indices, weights sum to the scaling factor, selection by corrected scores,
weights from raw scores); SwiGLU/SiTU against their closed forms at chosen points
(silu(0)=0, silu(x)->x for large x, situ's tanh saturation at +-beta); the expert FFN
against a brute-force per-row loop; the layer against a loop over experts.  The latent
layer: with identity down/up projections and unit norm weights it equals the normalised
plain layer; the routed scaling factor cancels in the normalisation (eps = 0); it is
linear in the up projection; a planted swap of normalisation and up projection fails.
"""
from __future__ import annotations

import numpy as np

from concurrent.futures import ThreadPoolExecutor

from .mxfp4 import decode_mxfp4, decode_mxfp4_f64


def sigmoid(g: np.ndarray) -> np.ndarray:
    """Overflow-free logistic: 1/(1+e^-g) == (1 + tanh(g/2)) / 2."""
    return 0.5 * (1.0 + np.tanh(0.5 * np.asarray(g, dtype=np.float64)))


def silu(g: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float64)
    return g * sigmoid(g)


def situ(g: np.ndarray, u: np.ndarray, beta: float, linear_beta: float | None) -> np.ndarray:
    """``beta*tanh(g/beta)*sigmoid(g) * linear_beta*tanh(u/linear_beta)``."""
    g = np.asarray(g, dtype=np.float64)
    u = np.asarray(u, dtype=np.float64)
    a = beta * np.tanh(g / beta) * sigmoid(g)
    if linear_beta is not None:
        u = linear_beta * np.tanh(u / linear_beta)
    return a * u


def activation(g, u, kind: str = "silu", beta: float = 1.0, linear_beta=None):
    if kind == "silu":
        return silu(g) * np.asarray(u, dtype=np.float64)
    if kind == "situ":
        return situ(g, u, beta, linear_beta)
    raise ValueError(kind)


def topk_lowest_index(scores: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest entries per row, largest first, ties to the lower index."""
    s = np.asarray(scores, dtype=np.float64)
    order = np.lexsort((np.broadcast_to(np.arange(s.shape[-1]), s.shape), -s), axis=-1)
    return order[..., :k]


def route_softmax(x, router_w, k: int, renormalize: bool = True, scaling: float = 1.0):
    """x [T, H], router_w [E, H] -> (idx [T, k], weights [T, k], probs [T, E], logits)."""
    logits = np.asarray(x, np.float64) @ np.asarray(router_w, np.float64).T
    z = logits - logits.max(axis=-1, keepdims=True)
    e = np.exp(z)
    probs = e / e.sum(axis=-1, keepdims=True)
    idx = topk_lowest_index(probs, k)
    w = np.take_along_axis(probs, idx, axis=-1)
    if renormalize and k > 1:
        w = w / (w.sum(axis=-1, keepdims=True) + 1e-20)
    return idx, w * scaling, probs, logits


def route_sigmoid_bias(x, router_w, bias, k: int, renormalize: bool = True,
                       scaling: float = 1.0):
    """The reference router (``k3ref/layers.py:214-224``)."""
    logits = np.asarray(x, np.float64) @ np.asarray(router_w, np.float64).T
    raw = sigmoid(logits)
    corrected = raw + np.asarray(bias, np.float64)[None, :]
    idx = topk_lowest_index(corrected, k)
    w = np.take_along_axis(raw, idx, axis=-1)
    if renormalize and k > 1:
        w = w / (w.sum(axis=-1, keepdims=True) + 1e-20)
    return idx, w * scaling, raw, corrected


def dense_ffn(x, wg, wu, wd, kind="silu", beta=1.0, linear_beta=None):
    """Expert FFN on already-dense (float) weights [I, H], [I, H], [H, I]."""
    x = np.asarray(x, np.float64)
    g = x @ np.asarray(wg, np.float64).T
    u = x @ np.asarray(wu, np.float64).T
    a = activation(g, u, kind, beta, linear_beta)
    return a @ np.asarray(wd, np.float64).T, g, u, a


def expert_ffn(x, gate, up, down, kind="silu", beta=1.0, linear_beta=None):
    """One MXFP4 expert; ``gate``/``up``/``down`` are ``(packed, scales)`` pairs."""
    return dense_ffn(x, decode_mxfp4(*gate), decode_mxfp4(*up), decode_mxfp4(*down),
                     kind, beta, linear_beta)


def moe_layer(x, idx, weights, experts, shared=None, kind="silu", beta=1.0,
              linear_beta=None, workers: int = 1):
    """Weighted sum of routed experts (+ shared expert on the same hidden state).

    ``experts[e]`` is ``(gate, up, down)`` of (packed, scales) pairs; ``shared`` is
    ``(wg, wu, wd)`` of dense float weights or None.  Each expert's tokens are gathered and
    its output scattered back as in ``k3ref/layers.py:252-256``; the weighted outputs are
    added to ``y`` in ascending expert id.  ``workers > 1`` computes the experts' outputs
    on that many threads (for full-size layers whose experts are all distinct; the sums are
    still taken in ascending id, so the result does not depend on ``workers``).
    """
    x = np.atleast_2d(np.asarray(x, np.float64))
    idx = np.atleast_2d(idx)
    weights = np.atleast_2d(weights)
    y = np.zeros((x.shape[0], x.shape[1]), np.float64)
    ids = sorted({int(v) for v in idx.reshape(-1)})

    def routed(e, dense_w):
        tok, slot = np.nonzero(idx == e)
        out = dense_ffn(x[tok], *dense_w, kind=kind, beta=beta, linear_beta=linear_beta)[0]
        return tok, out * weights[tok, slot][:, None]

    if workers > 1:
        def one(e):
            return routed(e, tuple(decode_mxfp4_f64(*pair) for pair in experts[e]))
        with ThreadPoolExecutor(max_workers=workers) as pool:
            parts = list(pool.map(one, ids))
    else:
        # expert ids that share one weight tuple (tests alias them) decode it once; the cache
        # holds the tuple itself, so its id cannot be reused by another object meanwhile
        dense = {}
        parts = []
        for e in ids:
            ex = experts[e]
            if id(ex) not in dense:
                dense[id(ex)] = (ex, tuple(decode_mxfp4_f64(*pair) for pair in ex))
            parts.append(routed(e, dense[id(ex)][1]))
    for tok, contrib in parts:
        y[tok] += contrib
    if shared is not None:
        y += dense_ffn(x, *shared, kind=kind, beta=beta, linear_beta=linear_beta)[0]
    return y


def rmsnorm(x, w, eps: float):
    """KimiRMSNorm (``ops.py:11-14``): ``w * x / sqrt(mean(x^2) + eps)`` over the last axis."""
    x = np.asarray(x, np.float64)
    return np.asarray(w, np.float64) * (x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps))


def latent_moe(x, router_w, bias, down_w, up_w, norm_w, experts, shared, k: int,
               renormalize: bool = True, scaling: float = 1.0, beta: float = 1.0,
               linear_beta=None, eps: float = 1e-5, kind: str = "situ", h_bf16: bool = False,
               workers: int = 1):
    """K3's routed layer (``moe.py:110-132``).

    x [T, H]; router_w [E, H] and bias [E] (sigmoid + bias routing); down_w [L, H] and
    up_w [H, L] the latent projections; norm_w [L]; ``experts[e]`` = (gate, up, down)
    (packed, scales) pairs of latent-width experts; ``shared`` = (wg, wu, wd) dense or
    None.  ``h_bf16`` rounds the latent state to bf16, as the reference's bf16 matmul
    ``flat @ self.down.T`` does (``moe.py:117``); ``workers`` is ``moe_layer``'s.
    Returns (y [T, H], idx, weights)."""
    x = np.atleast_2d(np.asarray(x, np.float64))
    idx, w, _, _ = route_sigmoid_bias(x, router_w, bias, k, renormalize, scaling)
    h = x @ np.asarray(down_w, np.float64).T
    if h_bf16:
        from .mxfp4 import bf16_round
        h = bf16_round(h.astype(np.float32)).astype(np.float64)
    y = moe_layer(h, idx, w, experts, None, kind, beta, linear_beta, workers)
    y = rmsnorm(y, norm_w, eps) @ np.asarray(up_w, np.float64).T
    if shared is not None:
        y = y + dense_ffn(x, *shared, kind=kind, beta=beta, linear_beta=linear_beta)[0]
    return y, idx, w
