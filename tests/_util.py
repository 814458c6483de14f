"""Shared test helpers: seeded inputs, numpy <-> torch bf16 / packed conversions."""

from __future__ import annotations

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
