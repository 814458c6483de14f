"""Shared test helpers: seeded inputs, numpy <-> torch bf16 / packed conversions."""

from __future__ import annotations

import math

import numpy as np

from oracle.quant_ref import bf16_bits, bf16_from_bits, bf16_round


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def randn_bf16(r: np.random.Generator, *shape, scale: float = 1.0) -> np.ndarray:
    """bf16-valued fp32 array ~ N(0, scale^2)."""
    return bf16_round((r.standard_normal(shape) * scale).astype(np.float32))


def to_dev_bf16(a: np.ndarray, device):
    import torch

    bits = bf16_bits(np.asarray(a, dtype=np.float32))
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(device)


def from_dev_bf16(t) -> np.ndarray:
    import torch

    bits = t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    return bf16_from_bits(bits)


def to_dev_packed(w: np.ndarray, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(w, dtype=np.uint32).view(np.int32).copy()).to(device)


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def rms(a) -> float:
    a = np.asarray(a, np.float64)
    return float(np.sqrt(np.mean(a * a)))


def assert_rms_close(got, ref, tol: float = 2e-2, what: str = ""):
    """The acceptance bar: max|got - ref| <= tol * RMS(ref)."""
    err, r = max_abs(got, ref), rms(ref)
    assert err <= tol * r, f"{what}: max|err| {err:.4g} > {tol} * RMS {r:.4g}"
    return err, r


ROPE_KAT_P = (1, 17, 16384)
# bf16 output rounding (2^-9 relative) plus the fp32 angle at p = 16384 (~1e-3 rad)
ROPE_KAT_TOL = 4e-3


def rope_kat_errors(rope_fn, D: int, base: float) -> float:
    """Largest deviation of ``rope_fn(x [1, 1, D], pos [1], base)`` from the closed form of
    non-traditional RoPE (dflash_model.py:187-194, ``traditional=False``): the unit vector e_i
    (i < D/2) at position p becomes cos(p*theta_i) e_i + sin(p*theta_i) e_{i+D/2},
    theta_i = base^(-2i/D), every other coordinate 0. i in {0, 1, D/4, D/2 - 1}, p in
    ``ROPE_KAT_P``; the angles come from float64 ``math``, independent of the oracle."""
    worst = 0.0
    for i in sorted({0, 1, D // 4, D // 2 - 1}):
        x = np.zeros((1, 1, D), np.float32)
        x[..., i] = 1.0
        theta = base ** (-2.0 * i / D)
        for p in ROPE_KAT_P:
            y = np.asarray(rope_fn(x, [p], base), np.float64).reshape(D)
            want = np.zeros(D)
            want[i] = math.cos(p * theta)
            want[i + D // 2] = math.sin(p * theta)
            worst = max(worst, float(np.abs(y - want).max()))
    return worst
