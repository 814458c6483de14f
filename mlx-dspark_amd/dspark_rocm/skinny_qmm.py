"""Skinny quantized matmul: the verify-window qmm behind the reference's ``skinny_qmm`` calls.

Same entry points and argument meaning as the reference module (skinny_qmm.py:174-265):
``fits(mod)``, ``plan(rows, n, k, bits)``, ``qmm(x2, weight, scales, biases, bits)``,
``call(mod, x, rows)`` and the ``WINDOW`` of rows served per quantization width. The kernel is
``dspark_qmm_affine`` (libdspark_rocm.so, gfx950 MFMA): it serves M = 1..16 at both widths,
so the window covers the whole verify range (the reference's Metal kernel starts at M = 5/6
because Apple's stock qmv wins below that; here there is no faster stock path to hand off to).

Launch refusals surface as ``DsparkError`` (the reference raises mlx's ValueError mentioning
"threadgroup"); :func:`is_threadgroup_refusal` recognises both, so a caller's fall-back logic
(small_m_qmm.measure_shapes) reads the same. There is no split-K cap to lower on MI355X — the
workgroup size is fixed at 256 threads — so ``s_cap``/``set_s_cap`` are kept only as the
recorded value the calibration caches with its verdicts.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib, ops

GROUP = 64
RT_MAX = 1                              # 16-row tiles per workgroup (one MFMA row tile)
WINDOW = {4: (1, 16), 8: (1, 16)}       # rows served per quantization width
S_MAX = 32                              # most K slices a launch splits into
_s_cap = S_MAX


def s_cap() -> int:
    return _s_cap


def set_s_cap(n: int) -> None:
    """Recorded split cap (kept for the calibration cache's schema; the launch geometry on
    MI355X never needs lowering)."""
    global _s_cap
    _s_cap = max(1, min(S_MAX, int(n)))


def fits(mod) -> bool:
    """The layout the kernel reads (skinny_qmm.py:174-181): 4- or 8-bit affine with biases,
    groups of 64, bf16 scales, K % 64 == 0. Any N >= 1 (rows past N are clamped in-kernel)."""
    w = getattr(mod, "weight", None)
    if w is None or getattr(mod, "biases", None) is None:
        return False
    bits = int(getattr(mod, "bits", 0))
    return (bits in WINDOW and int(getattr(mod, "group_size", 0)) == GROUP
            and getattr(mod, "mode", "affine") == "affine" and w.dim() == 2 and w.dtype == torch.int32
            and mod.scales.dtype == torch.bfloat16 and mod.biases.dtype == torch.bfloat16
            and (int(w.shape[1]) * 32 // bits) % GROUP == 0)


def is_threadgroup_refusal(e: BaseException) -> bool:
    """A launch the library refused for its geometry (shape/unsupported/workspace status), or
    mlx's own threadgroup-size refusal text."""
    if isinstance(e, _lib.DsparkError):
        return e.status in (-2, -4, -6)
    msg = str(e).lower()
    return "thread group" in msg or "threadgroup" in msg


def geometry(n: int, k: int, rows: int = 16, bits: int = 8) -> tuple[int, int]:
    """``(strips, S)``: 64-row output strips and K slices the launch uses for [n, k]."""
    p = plan(rows, n, k, bits)
    return p["strips"], p["slices"]


def plan(rows: int, n: int, k: int, bits: int, dtype=torch.bfloat16) -> dict:
    """Launch plan of ``rows`` x [n, k] as the library will run it (host query, no GPU work):
    K slices, groups per slice, 64-row strips, workgroups and workspace bytes."""
    if dtype != torch.bfloat16:
        raise ValueError(f"qmm: x dtype {dtype} (bfloat16 only)")
    lib = _lib.load()
    out = (ctypes.c_int32 * 4)()
    _lib.check("dspark_qmm_affine_plan", lib.dspark_qmm_affine_plan(rows, k, n, bits, GROUP, out))
    return {"rows": rows, "n": n, "k": k, "bits": bits, "slices": out[0], "groups_per_slice": out[1],
            "strips": out[2], "workgroups": out[3],
            "workspace_bytes": int(lib.dspark_qmm_affine_workspace(rows, k, n, bits, GROUP))}


def qmm(x2: torch.Tensor, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, bits: int,
        _plan=None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``x2 [rows, K] @ dequant(W)^T`` for gs64 affine 4/8-bit ``W`` -> ``[rows, N]`` (bf16)."""
    return ops.quantized_matmul(x2, weight, scales, biases, bits=bits, group_size=GROUP, out=out)


def call(mod, x: torch.Tensor, rows: int) -> torch.Tensor:
    """``QuantizedLinear(x)`` through the kernel: leading dims flattened to ``rows``, reshaped
    back, the module's ``bias`` added. The plan is cached on the module per (rows, s_cap) as
    in the reference (its per-call Python cost matters at ~370 linears per verify)."""
    plans = mod.__dict__.get("_dspark_skinny")
    if plans is None:
        plans = {}
        object.__setattr__(mod, "_dspark_skinny", plans)
    k = x.shape[-1]
    key = (rows, _s_cap)
    if key not in plans:
        plans[key] = plan(rows, int(mod.weight.shape[0]), int(k), int(mod.bits), x.dtype)
    y = qmm(x.reshape(rows, k), mod.weight, mod.scales, mod.biases, int(mod.bits), _plan=plans[key])
    y = y.reshape(*x.shape[:-1], y.shape[-1])
    if getattr(mod, "bias", None) is not None:
        y = y + mod.bias.to(y.dtype)
    return y
