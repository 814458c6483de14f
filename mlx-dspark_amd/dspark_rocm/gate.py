"""Load-time gates: the numerics check and the speed race a kernel must pass before a dispatch
scope routes a shape to it (the reference gates every kernel this way: small_m_qmm.py:142-230,
multirow_attn.py:404-488).

Timing is by HIP events on the current stream. Calls on one stream execute in issue order, so
a chain needs no data dependency between calls to be timed end to end; it rotates over several
same-shape operands (a model's layers, several KV sets) so their bytes come from HBM and not
from the last call's cache lines. Each side of a race is timed twice after a warm-up pass and
the faster of the two is kept, which removes one-off stalls of either path.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Sequence

import torch


def chain_ms(calls: Sequence[Callable[[], object]], repeat: int = 3) -> float:
    """Milliseconds per call of ``calls`` issued back to back, ``repeat`` times over, between
    two HIP events (after one untimed pass)."""
    for c in calls:
        c()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(repeat):
        for c in calls:
            c()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / (repeat * len(calls))


def speedup(stock: Sequence[Callable[[], object]], kernel: Sequence[Callable[[], object]], repeat: int = 3) -> float:
    """How many times faster the kernel chain runs than the stock chain (> 1: the kernel wins)."""
    t_stock = min(chain_ms(stock, repeat) for _ in range(2))
    t_kernel = min(chain_ms(kernel, repeat) for _ in range(2))
    return t_stock / t_kernel


def max_abs_diff(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.float() - b.float()).abs().max())


@dataclass(frozen=True)
class Bar:
    """A race requirement: at ``rows`` rows the kernel must be at least ``min_speedup`` times
    as fast as the stock path."""
    rows: int
    min_speedup: float

    def met(self, ratio: float) -> bool:
        return ratio >= self.min_speedup


def winning_tail(wins: Sequence[bool]) -> int | None:
    """Index where the run of wins that reaches the end of ``wins`` begins (a sweep ordered by
    size: the smallest size from which the kernel keeps winning), or None when the last entry
    loses."""
    start = len(wins)
    while start > 0 and wins[start - 1]:
        start -= 1
    return start if start < len(wins) else None
