"""Small-M quantized matmul for the verify window: dispatch, per-shape gate, scoped patch.

Mirrors the reference module (small_m_qmm.py) on torch: inside ``small_m_matmul(ids)`` the
``QuantizedLinear`` instances whose ``id`` is allowlisted send bf16 forwards with
``lo <= M <= hi`` rows (M = product of the leading dims) through :mod:`.skinny_qmm`
(the gfx950 kernel); every other call — unlisted instance, non-bf16 x, rows outside the
window, scope inactive — runs the module's stock path unchanged (small_m_qmm.py:71-80).

The patch is class-wide on ``QuantizedLinear.forward`` and restores the value it found on
entry, so it nests with other scopes holding the class (small_m_qmm.py:83-106; reference test
tests/test_small_m_qmm.py:159-171). :func:`measure_shapes` is the runtime gate
(small_m_qmm.py:142-230): numerics of the kernel against the stock path at M in
{lo, 8, 12, hi} (``max|d| <= 0.02 * max(max|ref|, 1)``) and a dependent-chain race over the
model's own same-shape layers (win >= 1.15x at M = 8 and 12, >= 0.97x at the bottom edge);
only shapes that pass are returned. Nothing there may raise: a kernel failure disables that
shape and the stock path stays.
"""

from __future__ import annotations

import contextlib
import time

import torch

from . import skinny_qmm as _sk
from .nn import QuantizedLinear

M4_MIN, M4_MAX = _sk.WINDOW[4]
M8_MIN, M8_MAX = _sk.WINDOW[8]
M_MIN, M_MAX = M8_MIN, M8_MAX

_orig_call = QuantizedLinear.forward
_active_ids: frozenset | None = None


def _in_features(mod) -> int:
    return int(mod.weight.shape[1]) * 32 // int(mod.bits)


def eligible(mod) -> bool:
    """Can this ``QuantizedLinear``'s shape/format run on the kernel at all?"""
    return isinstance(mod, QuantizedLinear) and _sk.fits(mod)


def shape_key(mod) -> str:
    return f"{_in_features(mod)}x{int(mod.weight.shape[0])}b{int(mod.bits)}"


def _rows(x) -> int:
    m = 1
    for d in x.shape[:-1]:
        m *= int(d)
    return m


def serves(mod, x) -> bool:
    """Would the active scope send this call to the kernel? (allowlisted instance, bf16 x,
    rows inside the width's window; small_m_qmm.py:71-80)"""
    if _active_ids is None or id(mod) not in _active_ids or x.dtype != torch.bfloat16:
        return False
    lo, hi = _sk.WINDOW[int(mod.bits)]
    return lo <= _rows(x) <= hi


def _mma_call(self, x):
    if serves(self, x) and x.is_cuda:
        return _sk.call(self, x, _rows(x))
    return _orig_call(self, x)


@contextlib.contextmanager
def small_m_matmul(ids: frozenset | None):
    """Route the allowlisted ``QuantizedLinear`` instances (by ``id``) through the kernel for
    forwards inside their width's window. ``None``/empty: a no-op scope."""
    global _active_ids
    if not ids or QuantizedLinear.forward is _mma_call:
        yield
        return
    prev = QuantizedLinear.forward
    _active_ids = frozenset(ids)
    QuantizedLinear.forward = _mma_call
    try:
        yield
    finally:
        QuantizedLinear.forward = prev
        _active_ids = None


def active() -> bool:
    return QuantizedLinear.forward is _mma_call


# ------------------------------------------------------------------ calibration

_CHAIN = 12
_EVALS = 4
_MIN_GAIN = 1.15
_EDGE_MIN = 0.97
_REL_TOL = 0.02


def _time_chain(step, x0) -> float:
    """Seconds per step of a DEPENDENT chain (each step's input depends on the previous output),
    median of the timed evaluations after a warm-up."""
    times = []
    for _ in range(_EVALS):
        x = x0
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in range(_CHAIN):
            y = step(x, t)
            x = x0 + (y.float().mean() * 1e-20).to(x0.dtype)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) / _CHAIN)
    rest = sorted(times[1:])
    return rest[len(rest) // 2]


def _kernel_rows(mod, x: torch.Tensor) -> torch.Tensor:
    return _sk.qmm(x, mod.weight, mod.scales, mod.biases, int(mod.bits))


def measure_shapes(*models, verbose: bool = False) -> list[str]:
    """Shape keys whose kernel path is numerically sane and faster than the stock path here."""
    groups: dict[str, list] = {}
    for model in models:
        if model is None:
            continue
        for _, mod in model.named_modules():
            if eligible(mod):
                groups.setdefault(shape_key(mod), []).append(mod)
    won: list[str] = []
    for key, mods in groups.items():
        try:
            on = _verdict(key, mods, verbose)
        except Exception as e:  # noqa: BLE001 - a kernel that will not launch is simply off
            if verbose:
                print(f"  small-M qmm: {key} rejected (kernel unavailable: {type(e).__name__}: {e})", flush=True)
            continue
        if on:
            won.append(key)
    return won


def numerics_ok(mod, seed: int = 0) -> bool:
    """The kernel against the stock path at M in {lo, 8, 12, hi}:
    ``max|kernel - stock| <= 0.02 * max(max|stock|, 1)`` (small_m_qmm.py:120, :199-205)."""
    K = _in_features(mod)
    lo, hi = _sk.WINDOW[int(mod.bits)]
    dev = mod.weight.device
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    for M in sorted({lo, 8, 12, hi}):
        x = (torch.randn((M, K), generator=g, device=dev) * 0.1).to(torch.bfloat16)
        ref = _orig_call(mod, x).float()
        if getattr(mod, "bias", None) is not None:
            ref = ref - mod.bias.float()
        got = _kernel_rows(mod, x).float()
        diff = (ref - got).abs().max().item()
        if not diff <= _REL_TOL * max(ref.abs().max().item(), 1.0):
            return False
    return True


def _verdict(key: str, mods: list, verbose: bool) -> bool:
    mod = mods[0]
    K = _in_features(mod)
    lo, hi = _sk.WINDOW[int(mod.bits)]
    dev = mod.weight.device
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    if not numerics_ok(mod):
        if verbose:
            print(f"  small-M qmm: {key} rejected (numerics)", flush=True)
        return False

    def race(M):
        x = (torch.randn((M, K), generator=g, device=dev) * 0.1).to(torch.bfloat16)

        def q_step(xx, t):
            return _orig_call(mods[t % len(mods)], xx)

        def k_step(xx, t):
            return _kernel_rows(mods[t % len(mods)], xx)

        tq = min(_time_chain(q_step, x), _time_chain(q_step, x))
        tk = min(_time_chain(k_step, x), _time_chain(k_step, x))
        return tq / tk

    g8, g12 = race(8), race(12)
    g_lo = race(lo) if lo < 6 else None
    on = g8 >= _MIN_GAIN and g12 >= _MIN_GAIN and (g_lo is None or g_lo >= _EDGE_MIN)
    if verbose:
        edge = f", M={lo} {g_lo:.2f}x" if g_lo is not None else ""
        print(f"  small-M qmm: {key} M=8 {g8:.2f}x, M=12 {g12:.2f}x{edge} ({'on' if on else 'off'})", flush=True)
    return on


def ids_for_shapes(shapes, *models) -> frozenset:
    """The instance allowlist for :func:`small_m_matmul`, from verified shape keys."""
    keys = set(shapes)
    out = set()
    for model in models:
        if model is None:
            continue
        for _, mod in model.named_modules():
            if eligible(mod) and shape_key(mod) in keys:
                out.add(id(mod))
    return frozenset(out)
