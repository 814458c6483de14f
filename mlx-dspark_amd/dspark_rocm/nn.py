"""Quantized layers holding the packed affine format (the torch analogue of mlx.nn's).

``QuantizedLinear`` plays the role of ``mlx.nn.QuantizedLinear`` in the reference: the verify
path's projections are instances of it, and ``small_m_qmm.small_m_matmul`` re-routes their
calls class-wide (small_m_qmm.py:71-106). Its own ``forward`` is the *stock* path — the
counterpart of ``mx.quantized_matmul`` that the reference falls through to outside the kernel
window (small_m_qmm.py:53): dequantize to fp32 and multiply, output in x's dtype. The stock
path serves shapes and dtypes the kernels do not (prefill widths, fp32 activations); the
verify window runs on the HIP kernel through the scope.

``QuantizedSwitchLinear`` holds one such matrix per expert (stacked on a leading axis), the
layout of mlx-lm's ``QuantizedSwitchLinear`` that ``SwitchGLU`` gathers from.
"""

from __future__ import annotations

import torch
from torch import nn

from . import quant

GROUP = quant.GROUP


class QuantizedLinear(nn.Module):
    """``y = x @ dequant(weight)^T (+ bias)`` over affine ``bits``-bit packed weights.

    weight int32 [out, in*bits/32] (uint32 bit patterns), scales/biases bf16 [out, in/64],
    optional bias [out]. ``mode`` is always "affine" (the only format the kernels read).
    """

    mode = "affine"

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 bias: torch.Tensor | None = None, *, bits: int, group_size: int = GROUP):
        super().__init__()
        if weight.dtype != torch.int32 or weight.dim() != 2:
            raise ValueError("weight: packed int32 [out, in*bits/32]")
        self.bits = int(bits)
        self.group_size = int(group_size)
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)
        if bias is not None:
            self.register_buffer("bias", bias)
        else:
            self.bias = None

    @property
    def in_features(self) -> int:
        return int(self.weight.shape[1]) * 32 // self.bits

    @property
    def out_features(self) -> int:
        return int(self.weight.shape[0])

    @classmethod
    def from_float(cls, w: torch.Tensor, bias: torch.Tensor | None = None, *, bits: int = 4,
                   group_size: int = GROUP) -> "QuantizedLinear":
        """Quantize a float [out, in] weight with this project's quantizer (quant.quantize)."""
        wq, s, b = quant.quantize(w, group_size, bits)
        return cls(wq, s, b, bias, bits=bits, group_size=group_size)

    @classmethod
    def random(cls, out_features: int, in_features: int, *, bits: int, device=None, generator=None,
               bias: bool = False) -> "QuantizedLinear":
        w, s, b = quant.random_quantized(out_features, in_features, bits, device=device, generator=generator)
        bb = None
        if bias:
            bb = (torch.randn(out_features, device=device, generator=generator) * 0.02).to(torch.bfloat16)
        return cls(w, s, b, bb, bits=bits)

    def stock(self, x: torch.Tensor) -> torch.Tensor:
        """The stock path: fp32 dequantize + matmul, result in x's dtype."""
        w = quant.dequantize(self.weight, self.scales, self.biases, self.group_size, self.bits)
        y = (x.reshape(-1, x.shape[-1]).to(torch.float32) @ w.t()).to(x.dtype)
        y = y.reshape(*x.shape[:-1], y.shape[-1])
        if self.bias is not None:
            y = y + self.bias.to(y.dtype)
        return y

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.stock(x)

    def __contains__(self, name: str) -> bool:
        """``"biases" in mod`` / ``"bias" in mod``, as the reference's fits() asks."""
        return getattr(self, name, None) is not None

    def __getitem__(self, name: str) -> torch.Tensor:
        return getattr(self, name)


class QuantizedSwitchLinear(nn.Module):
    """Per-expert affine matrices stacked: weight int32 [E, out, in*bits/32], scales/biases
    bf16 [E, out, in/64]."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *, bits: int,
                 group_size: int = GROUP):
        super().__init__()
        if weight.dtype != torch.int32 or weight.dim() != 3:
            raise ValueError("weight: packed int32 [E, out, in*bits/32]")
        self.bits = int(bits)
        self.group_size = int(group_size)
        self.register_buffer("weight", weight)
        self.register_buffer("scales", scales)
        self.register_buffer("biases", biases)

    @property
    def num_experts(self) -> int:
        return int(self.weight.shape[0])

    @classmethod
    def random(cls, experts: int, out_features: int, in_features: int, *, bits: int, device=None,
               generator=None) -> "QuantizedSwitchLinear":
        mats = [quant.random_quantized(out_features, in_features, bits, device=device, generator=generator)
                for _ in range(experts)]
        return cls(*(torch.stack([m[i] for m in mats]).contiguous() for i in range(3)), bits=bits)

    def triple(self):
        return self.weight, self.scales, self.biases

    def pack(self) -> None:
        """Hold the weights (also) in the packed expert form (``ops.moe_pack``), which the fused
        MoE block then reads; products are bit-identical."""
        from . import ops

        self.packed = ops.moe_pack(self.weight, bits=self.bits, group_size=self.group_size)

    def fused_triple(self):
        """(weights, scales, biases) for the fused block: the packed form when held."""
        packed = getattr(self, "packed", None)
        return (packed if packed is not None else self.weight), self.scales, self.biases
