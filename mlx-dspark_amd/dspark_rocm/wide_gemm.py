"""Prefill wide path: dequantize the weight once, in one HIP launch, then a GEMM.

The reference's ``wide_matmul`` (wide_gemm.py:173-232) on torch modules, with its contract
kept: inside the scope a ``QuantizedLinear`` forward at least ``min_rows`` wide (the rows are
the product of the leading dims, so a ``[1, L, K]`` prefill counts L) whose shape key is in the
verified allowlist takes the wide path, and the result is **bit-identical** to the stock path
for that shape; everything else runs the forward installed on entry, unchanged.

What the wide path replaces here. The stock path (:meth:`QuantizedLinear.stock`) dequantizes
with torch elementwise ops -- unpack through int64, convert, multiply, add: several passes over
an ``N x K`` fp32 tensor -- and then runs one fp32 GEMM. The wide path produces the same fp32
weight in one pass (``dspark_qmm_dequantize``: ``(scale * q) + bias``, each operation rounded
as torch rounds it, no fma contraction) and hands it to the same GEMM call with the same
operands, so the bits agree by construction; :func:`verified_shapes` still checks every shape
before it is allowed, as the reference does (wide_gemm.py:263-306), so a change to either side
turns a shape off instead of changing results. At prefill widths the win is the dequant chain
(its time scales with ``N*K``, the GEMM's with ``M*N*K``), so it is largest at the narrow end
of the prefill range; :func:`measure_crossover` races it per machine.

``exact=False`` is the bf16/fp16 variant: dequantize straight to x's dtype and run the GEMM in
that dtype on the matrix cores (fp32 accumulation), ~16x the fp32 peak. It rounds the weight to
x's dtype, so it is not bit-identical to the stock path: its shapes are verified against the
qmm numerics bar (``max|d| <= 0.02 * max(max|stock|, 1)``) instead, and it is off unless a
caller asks -- the role the reference gives its non-identical CPU co-prefill split
(wide_gemm.py:44-66). That split itself (a row share on the CPU stream over unified memory,
wide_gemm.py:130-170, :395-459) has no counterpart: a discrete MI355X has no CPU GEMM that adds
to 2.5 PFLOP/s of bf16 MFMA across PCIe.
"""

from __future__ import annotations

import contextlib
import math

import torch

from . import _scope, gate, ops
from .nn import QuantizedLinear

SAFE_MIN_ROWS = 256      # no scope routes forwards narrower than this (wide_gemm.py:95-96)
REL_TOL = 0.02           # numerics bar of the exact=False variant

_orig_call = QuantizedLinear.forward
_cfg = _scope.Slot()     # (min_rows, shapes or None, exact) while a scope is active
_below = _scope.Slot()   # the forward installed when the scope was entered


def _rows(x: torch.Tensor) -> int:
    """Rows the matmul sees: everything but the contracting dimension (wide_gemm.py:99-101)."""
    return math.prod(int(d) for d in x.shape[:-1])


def _in_features(mod) -> int:
    return int(mod.weight.shape[1]) * 32 // int(mod.bits)


def _eligible(mod) -> bool:
    """Affine 4/8-bit weights with biases in groups of 64 and scales of a dtype the dequantize
    kernel reads (wide_gemm.py:104-108); other modes are left alone rather than assumed."""
    return (isinstance(mod, QuantizedLinear) and getattr(mod, "mode", "affine") == "affine"
            and getattr(mod, "biases", None) is not None and int(mod.bits) in (4, 8)
            and int(mod.group_size) == 64 and mod.scales.dtype in ops.DEQUANT_DTYPES
            and mod.biases.dtype == mod.scales.dtype and _in_features(mod) % 64 == 0)


def shape_key(mod) -> str:
    """``"{in}x{out}x{bits}x{scale dtype}"``: the unit a verification verdict holds for
    (wide_gemm.py:254-259)."""
    return f"{_in_features(mod)}x{int(mod.weight.shape[0])}x{int(mod.bits)}x{str(mod.scales.dtype).split('.')[-1]}"


def wide_rows(mod, x: torch.Tensor, exact: bool = True) -> torch.Tensor:
    """The wide path's result for ``mod(x)`` (no routing decision): one dequantize launch,
    then the GEMM, then the module's bias, in the stock path's order of operations."""
    k = x.shape[-1]
    x2 = x.reshape(-1, k)
    if exact or x.dtype == torch.float32:
        w = ops.dequantize(mod.weight, mod.scales, mod.biases, bits=int(mod.bits), dtype=torch.float32)
        y = (x2.to(torch.float32) @ w.t()).to(x.dtype)
    else:
        w = ops.dequantize(mod.weight, mod.scales, mod.biases, bits=int(mod.bits), dtype=x.dtype)
        y = x2 @ w.t()
    y = y.reshape(*x.shape[:-1], y.shape[-1])
    if getattr(mod, "bias", None) is not None:
        y = y + mod.bias.to(y.dtype)
    return y


def serves(mod, x: torch.Tensor) -> bool:
    """Would the active scope send this forward to the wide path?"""
    cfg = _cfg.value
    if cfg is None or not x.is_cuda or not _eligible(mod):
        return False
    min_rows, shapes, _ = cfg
    if _rows(x) < min_rows:
        return False
    return shapes is None or shape_key(mod) in shapes


def _wide_call(self, x):
    if serves(self, x):
        return wide_rows(self, x, exact=_cfg.value[2])
    return (_below.value or _orig_call)(self, x)


@contextlib.contextmanager
def wide_matmul(min_rows: int | None, shapes=None, *, exact: bool = True):
    """Route ``QuantizedLinear`` forwards at least ``min_rows`` wide through dequantize-once +
    GEMM. ``None``/0 makes this a no-op, and so does a scope already installed (the inner
    one leaves the outer in place, wide_gemm.py:211-213). ``min_rows`` is raised to
    :data:`SAFE_MIN_ROWS`. ``shapes`` is the allowlist of :func:`shape_key` values that
    verified (``None`` allows every eligible shape: only correct when the caller verified
    them some other way). Exit restores the forward found on entry, so the scope nests with
    ``small_m_matmul`` (a prefill inside a decode loop)."""
    if not min_rows or active():
        yield
        return
    cfg = (max(int(min_rows), SAFE_MIN_ROWS), None if shapes is None else frozenset(shapes), bool(exact))
    with _cfg.holding(cfg), _below.holding(QuantizedLinear.forward), \
            _scope.replaced(QuantizedLinear, "forward", _wide_call):
        yield


def active() -> bool:
    return QuantizedLinear.forward is _wide_call


# ------------------------------------------------------------------ calibration

def _network(model):
    """Where a model keeps its modules: a wrapper holding its network as ``.model`` is searched
    there (wide_gemm.py:235-244)."""
    return getattr(model, "model", model)


def quantized_linears(*models):
    """Every eligible ``QuantizedLinear`` in the given models (target, drafter, ...), model by
    model in module order."""
    for net in (_network(m) for m in models if m is not None):
        if hasattr(net, "modules"):
            yield from filter(_eligible, net.modules())


def widest_quantized_linear(*models):
    """The eligible ``QuantizedLinear`` with the most weight words, the first of equals (the MLP
    projections that dominate prefill), or None for models without one (wide_gemm.py:247-251)."""
    return max(quantized_linears(*models), key=lambda mod: mod.weight.numel(), default=None)


def _probe_x(mod, M: int, gen: torch.Generator) -> torch.Tensor:
    return torch.randn((M, _in_features(mod)), generator=gen, device=mod.weight.device).to(mod.scales.dtype)


def _agrees(mod, M: int, exact: bool = True, seed: int = 0, draws: int = 2) -> bool:
    """Whether the wide path gives the stock path's result for this weight at ``M`` rows on
    ``draws`` random inputs: bit for bit, or (``exact=False``) within the qmm bar. One lucky
    match proves little, hence two draws by default (wide_gemm.py:262-280)."""
    gen = torch.Generator(device=mod.weight.device)
    gen.manual_seed(seed + M)

    def one_draw() -> bool:
        x = _probe_x(mod, M, gen)
        stock, wide = _orig_call(mod, x), wide_rows(mod, x, exact=exact)
        if stock.shape != wide.shape or not bool(torch.isfinite(wide.float()).all()):
            return False
        if exact:
            return torch.equal(stock, wide)
        return gate.max_abs_diff(stock, wide) <= REL_TOL * max(float(stock.float().abs().max()), 1.0)

    return all(one_draw() for _ in range(draws))


def _verifies(mod, rows, exact: bool) -> bool:
    try:
        return all(_agrees(mod, M, exact) for M in rows)
    except Exception:  # noqa: BLE001 - a shape the kernel refuses stays on the stock path
        return False


def verified_shapes(models, min_rows: int, widths: tuple[int, ...] = (512, 1024, 2048), *,
                    exact: bool = True) -> list[str]:
    """Shape keys across ``models`` whose wide path agrees with the stock path at ``min_rows``
    and at each of ``widths``, checked once per key on its first module, in first-seen order
    (wide_gemm.py:283-306): the per-shape allowlist of the scope."""
    first: dict[str, object] = {}
    for mod in quantized_linears(*models):
        first.setdefault(shape_key(mod), mod)
    rows = (min_rows, *widths)
    return [key for key, mod in first.items() if _verifies(mod, rows, exact)]


def _wide_wins(lin, M: int, gen: torch.Generator, exact: bool, margin: float) -> bool:
    """Whether the wide path beats the stock path by ``margin`` at ``M`` rows (HIP events over
    back-to-back calls, best of three)."""
    x = _probe_x(lin, M, gen)
    t_stock = min(gate.chain_ms([lambda: _orig_call(lin, x)]) for _ in range(3))
    t_wide = min(gate.chain_ms([lambda: wide_rows(lin, x, exact=exact)]) for _ in range(3))
    return t_stock > t_wide * (1.0 + margin)


def measure_crossover(*models, widths: tuple[int, ...] = (256, 512, 1024, 2048), margin: float = 0.02,
                      exact: bool = True) -> tuple[int, list[str]] | None:
    """``(min_rows, verified shape keys)`` for this machine and models, or None when the path
    stays off: nothing quantized, never faster, or no shape verifies (wide_gemm.py:337-376).

    The widest weight is raced at every width (widths under :data:`SAFE_MIN_ROWS` never take the
    path); ``min_rows`` is where the run of winning widths that reaches the widest one starts,
    and the shapes are those that verify there and at every wider width."""
    lin = widest_quantized_linear(*models)
    if lin is None:
        return None
    gen = torch.Generator(device=lin.weight.device)
    gen.manual_seed(1)
    wins = [M >= SAFE_MIN_ROWS and _wide_wins(lin, M, gen, exact, margin) for M in widths]
    start = gate.winning_tail(wins)
    if start is None:
        return None
    keys = verified_shapes(models, int(widths[start]), widths=tuple(widths[start + 1:]), exact=exact)
    return (int(widths[start]), keys) if keys else None
