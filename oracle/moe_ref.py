"""MoE routing and the grouped expert MLP.

The reference reaches these through mlx-lm (third-party, not in the reference tree; floor
``mlx-lm>=0.31.3``, pyproject.toml:19-28): SparseMoeBlock routing and SwitchGLU over
``mx.gather_qmm``. Its published algorithm, restated:

    gates  = softmax(logits, precise=True)        # fp32 math, result in the input dtype (bf16)
    inds   = argpartition(-gates, kth=k-1)[..., :k]
    scores = take_along_axis(gates, inds); scores /= scores.sum(-1)   # norm_topk_prob, bf16 ops
    y      = down(silu(gate(x)) * up(x)) per (token, expert) pair     # SwitchGLU, gather_qmm
    out    = (y * scores[..., None]).sum(-2)

Order rule (argpartition's order is unspecified): experts ranked by logit descending, then
expert id ascending — softmax is monotone, so this is one of argpartition's admissible answers
and it is exact. The elementwise ops round to bf16 after each op (mlx bf16 semantics):
h = bf16(bf16(g * bf16(sigmoid(g))) * u) with g, u the bf16 qmm outputs; the weighted
combine sums bf16(score * y) in fp32, slot order.

Parity with MLX bits is unpinned (mlx is not installed); the restatement is pinned by brute
force (sorting with Python's sorted(), per-pair qmm via dequantize-and-matmul) and invariants
(tests/test_oracle_moe.py).
"""

from __future__ import annotations

import numpy as np

from .qmm_ref import qmm_f64
from .quant_ref import bf16_round


def route(logits: np.ndarray, k: int, renorm: bool = True):
    """logits [M, E] (bf16 values) -> (inds int32 [M, k], scores bf16-valued fp32 [M, k])."""
    x = np.asarray(logits, dtype=np.float32)
    M, E = x.shape
    inds = np.empty((M, k), dtype=np.int32)
    scores = np.empty((M, k), dtype=np.float32)
    for t in range(M):
        xt = x[t].astype(np.float64)
        e = np.exp(xt - xt.max())
        gates = bf16_round((e / e.sum()).astype(np.float32))
        order = sorted(range(E), key=lambda j: (-x[t, j], j))[:k]
        inds[t] = order
        g = gates[order]
        if renorm:
            denom = bf16_round(np.float32(np.sum(g, dtype=np.float32)))
            g = bf16_round((g / denom).astype(np.float32))
        scores[t] = g
    return inds, scores


def bucket(inds: np.ndarray, E: int):
    """(token, slot) pairs p = t*k + j sorted by expert, stable in p.
    Returns (offsets [E+1], sorted_pairs [P], pair_pos [P])."""
    flat = np.asarray(inds).reshape(-1)
    order = np.argsort(flat, kind="stable").astype(np.int32)
    counts = np.bincount(flat, minlength=E)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    pos = np.empty_like(order)
    pos[order] = np.arange(order.size, dtype=np.int32)
    return offsets, order, pos


def gather_qmm(x, rows, experts, w, scales, biases, bits: int) -> np.ndarray:
    """y[p] = x[rows[p]] @ dequant(w[experts[p]])^T, bf16-valued fp32 [P, N]."""
    x = np.asarray(x, dtype=np.float32)
    n = w.shape[1]
    y = np.empty((len(rows), n), dtype=np.float32)
    for p, (r, e) in enumerate(zip(rows, experts)):
        y[p] = bf16_round(qmm_f64(x[r:r + 1], w[e], scales[e], biases[e], bits).astype(np.float32))[0]
    return y


def sigmoid_bf16(g: np.ndarray) -> np.ndarray:
    return bf16_round((1.0 / (1.0 + np.exp(-np.asarray(g, dtype=np.float64)))).astype(np.float32))


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = bf16_round(g)
    u = bf16_round(u)
    return bf16_round(bf16_round(g * sigmoid_bf16(g)) * u)


def switch_glu(x, logits, wg, sg, bg, wu, su, bu, wd, sd, bd, k: int, bits: int, renorm: bool = True):
    """Routed expert MLP for M tokens -> (out bf16-valued fp32 [M, H], inds, scores)."""
    x = np.asarray(x, dtype=np.float32)
    M, H = x.shape
    inds, scores = route(logits, k, renorm)
    out = np.zeros((M, H), dtype=np.float32)
    for t in range(M):
        acc = np.zeros(H, dtype=np.float32)
        for j in range(k):
            e = int(inds[t, j])
            g = bf16_round(qmm_f64(x[t:t + 1], wg[e], sg[e], bg[e], bits).astype(np.float32))
            u = bf16_round(qmm_f64(x[t:t + 1], wu[e], su[e], bu[e], bits).astype(np.float32))
            h = swiglu(g, u)
            y = bf16_round(qmm_f64(h, wd[e], sd[e], bd[e], bits).astype(np.float32))[0]
            acc = (acc + bf16_round(scores[t, j] * y)).astype(np.float32)
        out[t] = bf16_round(acc)
    return out, inds, scores


def expert_bytes(I: int, H: int, bits: int) -> int:
    """Bytes of one expert's gate+up+down at gs 64 with bf16 scales and biases."""
    per_param = bits / 8 + 4 / 64
    return int(3 * I * H * per_param)
