"""Row-split attention: a wide verify SDPA computed as several narrow sub-calls.

The reference uses this to step around a slow multi-row path of its stock attention
(sdpa_split.py:1-23, entry points :38-134). It is exact per row because every query row's
output depends only on that row and the keys it may see (sdpa_split.py:9-14), so cutting the
q_len rows into blocks and concatenating the block outputs changes only the reduction order.

Rows [a, b) of a ``"causal"`` call are the last ``b - a`` rows of a problem whose keys end at
``kv_len - q_len + b``: their sub-call keeps the "causal" string over that key prefix
(sdpa_split.py:84-87). An array mask of shape [..., q_len, kv_len] is cut to the block's rows;
one of shape [..., 1, kv_len] is shared by every block.

``sdpa_split(cfg)`` replaces :func:`dspark_rocm.fast.scaled_dot_product_attention` while
active. Blocks always call the stock function captured at import, never the replaced entry
point, so a split sub-call does not come back through any scope.
"""

from __future__ import annotations

import contextlib
from dataclasses import dataclass
from itertools import accumulate

import torch

from . import _scope, fast

_STOCK = fast.scaled_dot_product_attention


@dataclass(frozen=True)
class SplitConfig:
    """The split fires iff ``min_q <= q_len <= max_q`` and ``kv_len >= min_kv``; every
    sub-call then has at most ``max_chunk`` rows."""
    min_q: int = 6
    max_q: int = 15
    min_kv: int = 4096
    max_chunk: int = 5


def _partition(q_len: int, max_chunk: int) -> list[int]:
    """Block sizes: the fewest blocks of at most ``max_chunk`` rows, as even as possible,
    larger blocks first. Uses sum_{i<n} floor((q + i) / n) = q."""
    n = max(1, -(-q_len // max_chunk))
    return [(q_len + i) // n for i in range(n - 1, -1, -1)]


def _fires(cfg: SplitConfig, q_len: int, kv_len: int) -> bool:
    return cfg.min_q <= q_len <= cfg.max_q and kv_len >= cfg.min_kv


def split_sdpa(q, k, v, *, scale, mask=None, sinks=None, cfg: SplitConfig, _orig=None, **kw):
    """``scaled_dot_product_attention(q, k, v, ...)`` computed in row blocks when ``cfg``
    fires for this (q_len, kv_len); one unchanged call otherwise, or when an array mask's row
    dimension is neither 1 nor q_len."""
    sdpa = _orig or _STOCK
    q_len, kv_len = q.shape[-2], k.shape[-2]
    array_mask = isinstance(mask, torch.Tensor)
    mask_rows = (mask.shape[-2] if mask.dim() >= 2 else 1) if array_mask else None
    if not _fires(cfg, q_len, kv_len) or (array_mask and mask_rows not in (1, q_len)):
        return sdpa(q, k, v, scale=scale, mask=mask, sinks=sinks, **kw)
    sizes = _partition(q_len, cfg.max_chunk)
    ends = list(accumulate(sizes))
    pieces = []
    for stop, size in zip(ends, sizes):
        rows = slice(stop - size, stop)
        keys, values, block_mask = k, v, mask
        if isinstance(mask, str):
            visible = kv_len - q_len + stop
            keys, values = k[..., :visible, :], v[..., :visible, :]
        elif array_mask and mask_rows != 1:
            block_mask = mask[..., rows, :]
        pieces.append(sdpa(q[..., rows, :], keys, values, scale=scale, mask=block_mask, sinks=sinks, **kw))
    return torch.cat(pieces, dim=-2)


_config = _scope.Slot()


def _patched_call(q, k, v, *, scale, mask=None, sinks=None, **kw):
    cfg = _config.value
    if cfg is None:
        return _STOCK(q, k, v, scale=scale, mask=mask, sinks=sinks, **kw)
    return split_sdpa(q, k, v, scale=scale, mask=mask, sinks=sinks, cfg=cfg, _orig=_STOCK, **kw)


@contextlib.contextmanager
def sdpa_split(cfg: SplitConfig | None):
    """Route ``fast.scaled_dot_product_attention`` through :func:`split_sdpa` while active.
    A ``None`` config, or a split already installed, makes this scope a no-op."""
    if cfg is None or fast.scaled_dot_product_attention is _patched_call:
        yield
        return
    with _config.holding(cfg), _scope.replaced(fast, "scaled_dot_product_attention", _patched_call):
        yield


def patchable() -> bool:
    """Whether the attention entry point accepts a replacement (on this module it always does)."""
    return _scope.can_replace(fast, "scaled_dot_product_attention")
