"""Small-M affine quantized matmul, restated from the reference kernel (skinny_qmm.py:56-159):

    y[m, n] = sum_g ( scale[n,g] * P[m,n,g] + bias[n,g] * X[m,g] ),
    P[m,n,g] = sum_{j in g} q[n,j] * x[m,j],   X[m,g] = sum_{j in g} x[m,j]

(the factored form of skinny_qmm.py:138-145: ``acc = fma(bias, sum x, fma(scale, P, acc))``),
evaluated here in float64, then rounded to bfloat16 like the kernel's ``T(v)`` store
(skinny_qmm.py:158). A module-level Linear bias is added after (skinny_qmm.py:262-264).

Pinned by (tests/test_oracle_qmm.py): equality with dequantize-then-matmul (distributivity,
a different evaluation order); scales = 1 / biases = 0 against exact integer arithmetic;
one-hot x against a dequantized column; a pure-Python loop over the definition on K = 64,
N = 8; linearity in x; row-count invariance.
"""

from __future__ import annotations

import numpy as np

from .quant_ref import GROUP, bf16_round, unpack


def qmm_f64(x: np.ndarray, w: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int) -> np.ndarray:
    """x [M, K] (fp, typically bf16 values), packed w [N, K*bits/32] -> y fp64 [M, N]."""
    x = np.asarray(x, dtype=np.float64)
    m, k = x.shape
    q = unpack(w, bits).astype(np.float64)
    n = q.shape[0]
    assert q.shape[1] == k and k % GROUP == 0
    g = k // GROUP
    xg = x.reshape(m, g, GROUP)
    qg = q.reshape(n, g, GROUP)
    p = np.einsum("mgj,ngj->mng", xg, qg, optimize=True)
    sx = xg.sum(-1)
    s = np.asarray(scales, dtype=np.float64)
    b = np.asarray(biases, dtype=np.float64)
    return np.einsum("mng,ng->mn", p, s, optimize=True) + sx @ b.T


def qmm(x: np.ndarray, w: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int,
        bias: np.ndarray | None = None) -> np.ndarray:
    """bf16-valued fp32 output, as the kernel returns (x's dtype)."""
    y = qmm_f64(x, w, scales, biases, bits)
    out = bf16_round(y.astype(np.float32))
    if bias is not None:
        out = bf16_round(out + np.asarray(bias, dtype=np.float32))
    return out


def rms(a: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64)
    return float(np.sqrt(np.mean(a * a))) if a.size else 0.0


def within_rms_tol(got: np.ndarray, ref: np.ndarray, tol: float = 2e-2) -> tuple[bool, float, float]:
    """The acceptance bar: max|got - ref| <= tol * RMS(ref)."""
    err = float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64)))) if np.size(ref) else 0.0
    r = rms(ref)
    return err <= tol * r, err, r
