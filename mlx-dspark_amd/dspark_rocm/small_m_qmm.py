"""Small-M quantized matmul for the verify window: dispatch, per-shape gate, scoped patch.

The reference's entry points (small_m_qmm.py:57-243) on torch modules:

* ``small_m_matmul(ids)`` replaces ``QuantizedLinear.forward`` class-wide while active. A
  forward goes to the gfx950 kernel (:mod:`.skinny_qmm`) when the instance's ``id`` is in the
  allowlist, x is bf16 and its row count (product of the leading dims) lies in the width's
  ``WINDOW``; every other forward runs the method that was installed on entry, unchanged
  (small_m_qmm.py:71-80). Exit restores that method, so the scope nests with others holding
  the class (tests/test_small_m_qmm.py:159-171).
* ``measure_shapes(*models)`` is the load-time gate (small_m_qmm.py:142-230): per distinct
  shape, the kernel must agree with the stock path (``max|d| <= 0.02 * max(max|stock|, 1)``
  at M in {lo, 8, 12, hi}) and win a race over the model's own same-shape layers: 1.15x at
  M = 8 and 12, and no worse than 0.97x at the bottom of the window when it starts below 6.
  The race is :func:`dspark_rocm.gate.speedup` (HIP events). A shape whose kernel raises is
  off; nothing here raises.
"""

from __future__ import annotations

import contextlib
import math
from collections import defaultdict

import torch

from . import _scope, gate
from . import skinny_qmm as _sk
from .nn import QuantizedLinear

M4_MIN, M4_MAX = _sk.WINDOW[4]
M8_MIN, M8_MAX = _sk.WINDOW[8]
M_MIN, M_MAX = M8_MIN, M8_MAX

_orig_call = QuantizedLinear.forward
_allow = _scope.Slot()          # frozenset of module ids while a scope is active
_below = _scope.Slot()          # the forward installed when the scope was entered


def _in_features(mod) -> int:
    return int(mod.weight.shape[1]) * 32 // int(mod.bits)


def eligible(mod) -> bool:
    """Whether a module's shape and format can run on the kernel at all."""
    return isinstance(mod, QuantizedLinear) and _sk.fits(mod)


def shape_key(mod) -> str:
    """``"{in}x{out}b{bits}"``: modules with one key share a gate verdict."""
    return f"{_in_features(mod)}x{int(mod.weight.shape[0])}b{int(mod.bits)}"


def _rows(x) -> int:
    return math.prod(int(d) for d in x.shape[:-1])


def serves(mod, x) -> bool:
    """Would the active scope send this forward to the kernel?"""
    allow = _allow.value
    if not allow or id(mod) not in allow or x.dtype != torch.bfloat16:
        return False
    lo, hi = _sk.WINDOW[int(mod.bits)]
    return lo <= _rows(x) <= hi


def _mma_call(self, x):
    if x.is_cuda and serves(self, x):
        return _sk.call(self, x, _rows(x))
    return (_below.value or _orig_call)(self, x)


@contextlib.contextmanager
def small_m_matmul(ids: frozenset | None):
    """Send the allowlisted ``QuantizedLinear`` instances (by ``id``) to the kernel for
    forwards inside their width's window. An empty or ``None`` allowlist, or a scope already
    installed, makes this a no-op."""
    if not ids or active():
        yield
        return
    with _allow.holding(frozenset(ids)), _below.holding(QuantizedLinear.forward), \
            _scope.replaced(QuantizedLinear, "forward", _mma_call):
        yield


def active() -> bool:
    return QuantizedLinear.forward is _mma_call


# ------------------------------------------------------------------ load-time gate

_CHAIN = 12          # calls per timed chain (rotating over the shape's modules)
_EVALS = 4
_MIN_GAIN = 1.15
_EDGE_MIN = 0.97
_REL_TOL = 0.02


def _kernel_rows(mod, x: torch.Tensor) -> torch.Tensor:
    return _sk.qmm(x, mod.weight, mod.scales, mod.biases, int(mod.bits))


def _probe_x(K: int, M: int, gen: torch.Generator, device) -> torch.Tensor:
    return (0.1 * torch.randn((M, K), generator=gen, device=device)).to(torch.bfloat16)


def numerics_ok(mod, seed: int = 0) -> bool:
    """Kernel vs stock at M in {lo, 8, 12, hi}: ``max|kernel - stock| <= 0.02 * max(max|stock|, 1)``
    (the module's own bias, if any, is left out of both)."""
    K = _in_features(mod)
    lo, hi = _sk.WINDOW[int(mod.bits)]
    gen = torch.Generator(device=mod.weight.device)
    gen.manual_seed(seed)
    bias = getattr(mod, "bias", None)
    for M in sorted({lo, 8, 12, hi}):
        x = _probe_x(K, M, gen, mod.weight.device)
        stock = _orig_call(mod, x).float()
        if bias is not None:
            stock = stock - bias.float()
        scale = max(float(stock.abs().max()), 1.0)
        if not gate.max_abs_diff(_kernel_rows(mod, x), stock) <= _REL_TOL * scale:
            return False
    return True


def _bars(bits: int) -> list[gate.Bar]:
    lo = _sk.WINDOW[bits][0]
    bars = [gate.Bar(8, _MIN_GAIN), gate.Bar(12, _MIN_GAIN)]
    if lo < 6:
        bars.append(gate.Bar(lo, _EDGE_MIN))
    return bars


def _race(mods: list, rows: int, gen: torch.Generator) -> float:
    """Stock / kernel time at ``rows`` rows over chains rotating through ``mods``."""
    x = _probe_x(_in_features(mods[0]), rows, gen, mods[0].weight.device)
    seq = [mods[t % len(mods)] for t in range(_CHAIN)]
    return gate.speedup([lambda m=m: _orig_call(m, x) for m in seq],
                        [lambda m=m: _kernel_rows(m, x) for m in seq], repeat=_EVALS - 1)


def _shape_verdict(key: str, mods: list, verbose: bool) -> bool:
    if not numerics_ok(mods[0]):
        if verbose:
            print(f"  small-M qmm: {key} off (numerics)", flush=True)
        return False
    gen = torch.Generator(device=mods[0].weight.device)
    gen.manual_seed(0)
    results = [(bar, _race(mods, bar.rows, gen)) for bar in _bars(int(mods[0].bits))]
    on = all(bar.met(r) for bar, r in results)
    if verbose:
        detail = ", ".join(f"M={bar.rows} {r:.2f}x (>= {bar.min_speedup})" for bar, r in results)
        print(f"  small-M qmm: {key} {detail}: {'on' if on else 'off'}", flush=True)
    return on


def _by_shape(models) -> dict[str, list]:
    groups: dict[str, list] = defaultdict(list)
    for model in (m for m in models if m is not None):
        for mod in model.modules():
            if eligible(mod):
                groups[shape_key(mod)].append(mod)
    return groups


def measure_shapes(*models, verbose: bool = False) -> list[str]:
    """Shape keys whose kernel path agrees with the stock path and wins the race here."""
    won = []
    for key, mods in _by_shape(models).items():
        try:
            if _shape_verdict(key, mods, verbose):
                won.append(key)
        except Exception as e:  # noqa: BLE001 - a kernel that will not launch leaves the shape off
            if verbose:
                print(f"  small-M qmm: {key} off (kernel unavailable: {type(e).__name__}: {e})", flush=True)
    return won


def ids_for_shapes(shapes, *models) -> frozenset:
    """The instance allowlist for :func:`small_m_matmul`: every eligible module of ``models``
    whose shape key is in ``shapes``."""
    keys = set(shapes)
    return frozenset(id(mod) for key, mods in _by_shape(models).items() if key in keys for mod in mods)
