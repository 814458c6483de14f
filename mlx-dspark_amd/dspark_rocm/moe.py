"""Routed-expert MoE block on the gfx950 kernels: routing, ``gather_qmm``, SwitchGLU.

The reference reaches MoE targets through mlx-lm's qwen3_moe-style ``SparseMoeBlock`` and
``SwitchGLU`` / ``QuantizedSwitchLinear`` (third-party, not vendored; the reference routes
them at load.py:111-123 and counts their bytes at roofline.py:190-245). Semantics restated:

    gates  = softmax(router(x))                  fp32 math ("precise"), bf16 result
    inds   = top-k of gates per token            (mx.argpartition: order unspecified)
    scores = gates[inds]; scores /= sum(scores)  when norm_topk_prob
    y      = SwitchGLU(x, inds)                  down(silu(gate(x)) * up(x)) per (token, slot)
    out    = sum_j scores[j] * y[j]

``gather_qmm`` keeps mx.gather_qmm's arguments (x, w, scales, biases, lhs_indices,
rhs_indices, transpose, group_size, bits, sorted_indices): output ``p`` is
``x[lhs[p]] @ dequant(w[rhs[p]])^T``. SwitchGLU sorts the (token, slot) pairs by expert
when there are at least 64 of them (mlx-lm's threshold) and unsorts the result.

The tie rule of top-k here is (logit desc, expert id asc): deterministic, and one of the
orders argpartition may return. ``SparseMoeBlock.forward`` runs the whole block as one fused
call (``dspark_moe_switch_glu``: route, gate/up with SwiGLU, down, combine).
"""

from __future__ import annotations

import torch
from torch import nn

from . import ops
from .nn import QuantizedLinear, QuantizedSwitchLinear

SORT_THRESHOLD = 64


def route(logits: torch.Tensor, k: int, renorm: bool = True):
    """(inds int32 [M, k], scores bf16 [M, k]) of softmax top-k routing on the GPU."""
    lead = logits.shape[:-1]
    inds, scores = ops.moe_route(logits.reshape(-1, logits.shape[-1]), k, renorm=renorm)
    return inds.reshape(*lead, k), scores.reshape(*lead, k)


def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               lhs_indices: torch.Tensor | None = None, rhs_indices: torch.Tensor | None = None,
               transpose: bool = True, group_size: int = 64, bits: int = 4,
               sorted_indices: bool = False) -> torch.Tensor:
    """``out[p] = x[lhs[p]] @ dequant(w[rhs[p]])^T`` for every index p of ``rhs_indices``.

    x [..., M, K] bf16 (its leading dims flattened are what ``lhs_indices`` index; with no
    ``lhs_indices`` they broadcast against ``rhs_indices``), w packed [E, N, K*bits/32].
    Returns [*rhs_indices.shape, M, N]. ``sorted_indices``: the caller guarantees
    ``rhs_indices`` is already non-decreasing (the pairs arrive expert-sorted).
    """
    if not transpose:
        raise ValueError("gather_qmm: only transpose=True (weights [E, N, K]) is supported")
    if rhs_indices is None:
        raise ValueError("gather_qmm: rhs_indices (expert per output) is required")
    E, N = int(w.shape[0]), int(w.shape[1])
    K = int(x.shape[-1])
    M = int(x.shape[-2])
    xb = x.reshape(-1, M, K)
    experts = rhs_indices.reshape(-1).to(torch.int64)
    P = experts.numel()
    if lhs_indices is not None:
        lhs = torch.broadcast_to(lhs_indices, rhs_indices.shape).reshape(-1).to(torch.int64)
    elif xb.shape[0] == P:
        lhs = torch.arange(P, device=x.device)
    elif xb.shape[0] == 1:
        lhs = torch.zeros(P, dtype=torch.int64, device=x.device)
    else:
        lhs = torch.arange(xb.shape[0], device=x.device).reshape(
            *x.shape[:-2]).expand(*rhs_indices.shape).reshape(-1)
    if sorted_indices:
        order = torch.arange(P, device=x.device)
        se = experts
    else:
        se, order = torch.sort(experts, stable=True)
    counts = torch.bincount(se, minlength=E)
    offsets = torch.zeros(E + 1, dtype=torch.int32, device=x.device)
    offsets[1:] = torch.cumsum(counts, 0).to(torch.int32)
    # sorted position s covers rows lhs[order[s]] * M + r, r < M (each pair's M rows are
    # consecutive and share its expert)
    rows = (lhs[order].unsqueeze(1) * M + torch.arange(M, device=x.device).unsqueeze(0)).reshape(-1)
    offsets = offsets * M
    ys = ops.gather_qmm_sorted(xb.reshape(-1, K), w, scales, biases, offsets, row_index=rows.to(torch.int32),
                               bits=bits, group_size=group_size, rows=P * M)
    y = torch.empty_like(ys)
    y.view(P, M, N)[order] = ys.view(P, M, N)
    return y.reshape(*rhs_indices.shape, M, N)


def _gather_sort(x: torch.Tensor, indices: torch.Tensor):
    """Flatten the (token, slot) pairs and sort them by expert: (x rows of the sorted pairs,
    sorted expert ids, inverse order)."""
    k = indices.shape[-1]
    flat = indices.reshape(-1)
    idx, order = torch.sort(flat.to(torch.int64), stable=True)
    inv = torch.argsort(order)
    return x.reshape(-1, *x.shape[-2:])[order // k], idx, inv


class SwitchGLU(nn.Module):
    """``down(silu(gate(x)) * up(x))`` with per-(token, slot) experts (mlx-lm SwitchGLU)."""

    def __init__(self, gate_proj: QuantizedSwitchLinear, up_proj: QuantizedSwitchLinear,
                 down_proj: QuantizedSwitchLinear):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    @classmethod
    def random(cls, experts: int, hidden: int, intermediate: int, *, bits: int = 4, device=None, generator=None):
        return cls(QuantizedSwitchLinear.random(experts, intermediate, hidden, bits=bits, device=device, generator=generator),
                   QuantizedSwitchLinear.random(experts, intermediate, hidden, bits=bits, device=device, generator=generator),
                   QuantizedSwitchLinear.random(experts, hidden, intermediate, bits=bits, device=device, generator=generator))

    def pack(self) -> "SwitchGLU":
        """Pack the three projections' expert weights for the fused block (bit-identical
        products; the row-major weights stay for the unfused path)."""
        for lin in (self.gate_proj, self.up_proj, self.down_proj):
            lin.pack()
        return self

    def _proj(self, lin: QuantizedSwitchLinear, x, idx, sorted_indices):
        return gather_qmm(x, *lin.triple(), rhs_indices=idx, bits=lin.bits, group_size=lin.group_size,
                          sorted_indices=sorted_indices)

    def forward(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        """x [..., H] bf16, indices [..., k] -> [..., k, H]."""
        xe = x.unsqueeze(-2).unsqueeze(-2)               # [..., 1, 1, H]
        do_sort = indices.numel() >= SORT_THRESHOLD
        idx, inv = indices, None
        if do_sort:
            xe, idx, inv = _gather_sort(xe, indices)
        up = self._proj(self.up_proj, xe, idx, do_sort)
        gate = self._proj(self.gate_proj, xe, idx, do_sort)
        h = (gate * torch.sigmoid(gate)) * up             # mlx's silu: bf16 sigmoid, then mul, mul
        y = self._proj(self.down_proj, h, idx, do_sort)
        if do_sort:
            y = y[inv].reshape(*indices.shape, 1, y.shape[-1])
        return y.squeeze(-2)


class SparseMoeBlock(nn.Module):
    """qwen3_moe-style block: router ``gate`` (QuantizedLinear [E, H]), ``switch_mlp``."""

    def __init__(self, gate: QuantizedLinear, switch_mlp: SwitchGLU, *, top_k: int, norm_topk_prob: bool = True):
        super().__init__()
        self.gate, self.switch_mlp = gate, switch_mlp
        self.top_k = int(top_k)
        self.norm_topk_prob = bool(norm_topk_prob)

    def router_logits(self, x: torch.Tensor) -> torch.Tensor:
        return self.gate(x)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Fused block on the GPU: one route + gate/up + down + combine sequence."""
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1])
        logits = self.router_logits(x2)
        mlp = self.switch_mlp
        out, _, _ = ops.moe_switch_glu(x2, logits, mlp.gate_proj.fused_triple(), mlp.up_proj.fused_triple(),
                                       mlp.down_proj.fused_triple(), k=self.top_k, bits=mlp.gate_proj.bits,
                                       renorm=self.norm_topk_prob, group_size=mlp.gate_proj.group_size)
        return out.reshape(*lead, out.shape[-1])

    def forward_unfused(self, x: torch.Tensor) -> torch.Tensor:
        """The same block as separate steps (route, SwitchGLU via gather_qmm, weighted sum)."""
        logits = self.router_logits(x)
        inds, scores = route(logits, self.top_k, self.norm_topk_prob)
        y = self.switch_mlp(x, inds)                                   # [..., k, H]
        w = (scores.unsqueeze(-1).float() * y.float()).to(torch.bfloat16)
        return w.float().sum(dim=-2).to(x.dtype)
