"""Affine 4/8-bit packed format, restated from the reference kernel's unpacking
(skinny_qmm.py:95-119; A.1 "exact semantics"): element j of row n is field j % (32/bits) of
uint32 word j // (32/bits), bits [bits*f, bits*f + bits), low bits first; groups of 64 along K
share one scale and one bias: dequant(n, j) = scale[n, j//64] * q + bias[n, j//64].

Pinned by: hand KATs (0x76543210 at 4-bit -> 0..7; 0x04030201 at 8-bit -> 1,2,3,4), pack/unpack
round trips, and a pure-Python bit-loop cross-check (tests/test_oracle_quant.py).
"""

from __future__ import annotations

import numpy as np

GROUP = 64


def bf16_round(a: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bfloat16 (ties to even), returned as fp32 values."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(a), a, out).astype(np.float32)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """fp32 -> bfloat16 bit patterns (uint16), round to nearest even."""
    return (bf16_round(a).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack(q: np.ndarray, bits: int) -> np.ndarray:
    """integer q [N, K] in [0, 2^bits) -> uint32 words [N, K*bits/32]."""
    f = 32 // bits
    q = np.asarray(q, dtype=np.uint64)
    n, k = q.shape
    assert k % f == 0 and q.max(initial=0) < (1 << bits)
    shifts = (np.arange(f, dtype=np.uint64) * bits)
    return (q.reshape(n, k // f, f) << shifts).sum(axis=-1).astype(np.uint32)


def unpack(w: np.ndarray, bits: int) -> np.ndarray:
    """uint32 words [N, W] -> q [N, W*32/bits] (int64)."""
    f = 32 // bits
    w = np.asarray(w).astype(np.uint64) & 0xFFFFFFFF
    shifts = np.arange(f, dtype=np.uint64) * bits
    q = (w[..., None] >> shifts) & ((1 << bits) - 1)
    return q.reshape(*w.shape[:-1], -1).astype(np.int64)


def dequantize(w: np.ndarray, scales: np.ndarray, biases: np.ndarray, bits: int) -> np.ndarray:
    """packed [N, W] + fp scales/biases [N, K/64] -> fp64 [N, K]."""
    q = unpack(w, bits).astype(np.float64)
    n, k = q.shape
    s = np.asarray(scales, dtype=np.float64)
    b = np.asarray(biases, dtype=np.float64)
    return (q.reshape(n, k // GROUP, GROUP) * s[..., None] + b[..., None]).reshape(n, k)


def quantize(w: np.ndarray, bits: int):
    """fp [N, K] -> (uint32 packed, scales bf16-valued fp32, biases bf16-valued fp32).

    Same rule as the build's own quantizer: scale = (max - min)/(2^bits - 1), bias = min, both
    rounded to bf16, q = clip(round((w - bias)/scale)). (mx.quantize's exact choice is not
    reproducible without MLX and no kernel depends on it.)"""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    wg = w.reshape(n, k // GROUP, GROUP)
    lo, hi = wg.min(-1), wg.max(-1)
    levels = (1 << bits) - 1
    s = bf16_round(((hi - lo) / levels).astype(np.float32))
    b = bf16_round(lo)
    ss = np.where(s == 0, 1.0, s)
    q = np.clip(np.round((wg - b[..., None]) / ss[..., None]), 0, levels).astype(np.int64).reshape(n, k)
    return pack(q, bits), s, b


def random_packed(rng: np.random.Generator, n: int, k: int, bits: int, scale_std: float = 0.02):
    """Synthetic packed weights in the packed domain (uniform fields), with bf16-valued scales
    and biases shaped like an N(0, scale_std) weight's. Returns (w uint32, scales, biases) with
    scales/biases as fp32 arrays holding bf16 values."""
    words = rng.integers(0, 2**32, size=(n, k * bits // 32), dtype=np.uint64).astype(np.uint32)
    g = k // GROUP
    levels = (1 << bits) - 1
    span = 6.0 * scale_std
    s = bf16_round((span / levels) * (0.75 + 0.5 * rng.random((n, g))).astype(np.float32))
    b = bf16_round((-0.5 * span + 0.1 * scale_std * rng.standard_normal((n, g))).astype(np.float32))
    return words, s, b
