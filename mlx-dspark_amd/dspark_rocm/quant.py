"""Affine 4/8-bit group quantization: the packed-weight format the kernels read.

Format (the reference kernel's, skinny_qmm.py:95-119 and A.1 of its algorithm): ``w[n, k]``
becomes ``q[n, k]`` in ``[0, 2^bits)`` with ``dequant = scale[n, k // gs] * q + bias[n, k // gs]``;
``q[n, j]`` is field ``j % (32 // bits)`` (bits ``[bits*f, bits*f + bits)``, low bits first) of
uint32 word ``j // (32 // bits)`` of row ``n``. Scales and biases are bfloat16 ``[N, K // gs]``.

The quantizer here (round-to-nearest over the group's [min, max] range) is this project's own:
``mx.quantize``'s exact scale/bias choice is not reproducible without MLX, and nothing in the
kernels depends on how scales and biases were chosen. Tensors are torch tensors on any device;
packed words are stored as int32 (torch has no uint32 arithmetic) and reinterpreted by the kernel.
"""

from __future__ import annotations

import torch

GROUP = 64
BITS = (4, 8)


def _check(bits: int, group_size: int) -> None:
    if bits not in BITS:
        raise ValueError(f"bits={bits}: only 4 and 8 are supported")
    if group_size != GROUP:
        raise ValueError(f"group_size={group_size}: only 64 is supported")


def pack(q: torch.Tensor, bits: int) -> torch.Tensor:
    """``q`` integer [N, K] in [0, 2^bits) -> packed int32 [N, K*bits/32] (low bits first)."""
    if bits not in BITS:
        raise ValueError(f"bits={bits}")
    n, k = q.shape
    f = 32 // bits
    if k % f:
        raise ValueError(f"K={k} is not a multiple of {f}")
    qq = q.to(torch.int64).reshape(n, k // f, f)
    shifts = torch.arange(f, device=q.device, dtype=torch.int64) * bits
    words = (qq << shifts).sum(dim=-1)                       # < 2^32, exact in int64
    words = torch.where(words >= 2**31, words - 2**32, words)  # reinterpret as int32
    return words.to(torch.int32).contiguous()


def unpack(w: torch.Tensor, bits: int) -> torch.Tensor:
    """Packed int32/uint32 [N, W] -> integer q [N, W*32/bits] (int32)."""
    if bits not in BITS:
        raise ValueError(f"bits={bits}")
    f = 32 // bits
    ww = w.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(f, device=w.device, dtype=torch.int64) * bits
    q = (ww.unsqueeze(-1) >> shifts) & ((1 << bits) - 1)
    return q.reshape(w.shape[0], -1).to(torch.int32)


def quantize(w: torch.Tensor, group_size: int = GROUP, bits: int = 4):
    """fp weight [N, K] -> (packed int32 [N, K*bits/32], scales bf16 [N, K/gs], biases bf16).

    scale = (max - min) / (2^bits - 1), bias = min, both rounded to bf16 first; q is then
    round((w - bias) / scale) clamped to range, so ``scale*q + bias`` uses the stored values.
    """
    _check(bits, group_size)
    n, k = w.shape
    if k % group_size:
        raise ValueError(f"K={k} is not a multiple of {group_size}")
    wg = w.to(torch.float32).reshape(n, k // group_size, group_size)
    lo = wg.amin(dim=-1)
    hi = wg.amax(dim=-1)
    levels = (1 << bits) - 1
    scale = ((hi - lo) / levels).to(torch.bfloat16)
    bias = lo.to(torch.bfloat16)
    s32 = scale.to(torch.float32)
    s_safe = torch.where(s32 == 0, torch.ones_like(s32), s32)
    q = torch.round((wg - bias.to(torch.float32).unsqueeze(-1)) / s_safe.unsqueeze(-1))
    q = q.clamp_(0, levels).to(torch.int32).reshape(n, k)
    return pack(q, bits), scale.contiguous(), bias.contiguous()


def quantize_rows(x: torch.Tensor, bits: int, group_size: int = GROUP, dtype=torch.bfloat16):
    """Quantize the last dim of ``x`` [..., D] with the rule of :func:`quantize` (scales and
    biases rounded to ``dtype``): (words int32 [..., D*bits/32], scales [..., D/gs], biases)."""
    lead, d = x.shape[:-1], x.shape[-1]
    _check(bits, group_size)
    if d % group_size:
        raise ValueError(f"D={d} is not a multiple of {group_size}")
    xg = x.reshape(-1, d // group_size, group_size).to(torch.float32)
    lo, hi = xg.amin(dim=-1), xg.amax(dim=-1)
    levels = (1 << bits) - 1
    scale = ((hi - lo) / levels).to(dtype)
    bias = lo.to(dtype)
    s32 = scale.to(torch.float32)
    s_safe = torch.where(s32 == 0, torch.ones_like(s32), s32)
    q = torch.round((xg - bias.to(torch.float32).unsqueeze(-1)) / s_safe.unsqueeze(-1)).clamp_(0, levels)
    words = pack(q.to(torch.int32).reshape(-1, d), bits)
    return (words.reshape(*lead, d * bits // 32), scale.reshape(*lead, d // group_size),
            bias.reshape(*lead, d // group_size))


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int = GROUP,
               bits: int = 4) -> torch.Tensor:
    """Packed weights -> fp32 [N, K] (``scale*q + bias`` in fp32)."""
    _check(bits, group_size)
    q = unpack(w, bits).to(torch.float32)
    n, k = q.shape
    qg = q.reshape(n, k // group_size, group_size)
    out = qg * scales.to(torch.float32).unsqueeze(-1) + biases.to(torch.float32).unsqueeze(-1)
    return out.reshape(n, k)


def random_quantized(n: int, k: int, bits: int, *, generator: torch.Generator | None = None,
                     device="cpu", scale_std: float = 0.02):
    """Synthetic packed weights drawn directly in the packed domain (uniform fields, scales and
    biases shaped like an N(0, scale_std) weight's): cheap enough for multi-GB pools."""
    words_per_row = k * bits // 32
    g = k // GROUP
    w = torch.randint(-2**31, 2**31 - 1, (n, words_per_row), dtype=torch.int32, device=device,
                      generator=generator)
    levels = (1 << bits) - 1
    span = 6.0 * scale_std
    s = torch.full((n, g), span / levels, dtype=torch.float32, device=device)
    s = s * (0.75 + 0.5 * torch.rand((n, g), device=device, generator=generator))
    b = -0.5 * span + 0.1 * scale_std * torch.randn((n, g), device=device, generator=generator)
    return w, s.to(torch.bfloat16), b.to(torch.bfloat16)
