"""Split a wide-verify SDPA into narrow sub-calls (the reference's fallback path).

Mirrors sdpa_split.py: each query row's attention is independent, so computing the q_len rows
in balanced <= ``max_chunk``-row sub-calls and concatenating equals one call per row up to
reduction order (sdpa_split.py:9-14). For the string "causal" mask, chunk rows [off, off+p)
are the last rows of a shorter problem: they attend ``k[..., :kv_len - q_len + off + p]``
under the same "causal" rule (sdpa_split.py:84-87); array masks are sliced per row.

The scope ``sdpa_split(cfg)`` patches :func:`dspark_rocm.fast.scaled_dot_product_attention`
(the reference patches ``mx.fast.scaled_dot_product_attention``) and restores it on exit;
:mod:`.multirow_attn` installs over it and falls through to it.
"""

from __future__ import annotations

import contextlib
import math
from dataclasses import dataclass

import torch

from . import fast

_ORIG_SDPA = fast.scaled_dot_product_attention


@dataclass(frozen=True)
class SplitConfig:
    """Split fires iff ``min_q <= q_len <= max_q`` and ``kv_len >= min_kv``; ``max_chunk``
    bounds each sub-call's q_len."""
    min_q: int = 6
    max_q: int = 15
    min_kv: int = 4096
    max_chunk: int = 5


def _partition(q_len: int, max_chunk: int) -> list[int]:
    """Balanced split of ``q_len`` into ceil(q_len / max_chunk) chunks, larger chunks first."""
    n = max(1, math.ceil(q_len / max_chunk))
    base, rem = divmod(q_len, n)
    return [base + 1] * rem + [base] * (n - rem)


def split_sdpa(q, k, v, *, scale, mask=None, sinks=None, cfg: SplitConfig, _orig=None, **kw):
    """``scaled_dot_product_attention`` computed in row chunks when the gate fires; a single
    call (verbatim) otherwise."""
    orig = _orig or _ORIG_SDPA
    q_len = q.shape[-2]
    kv_len = k.shape[-2]
    if not (cfg.min_q <= q_len <= cfg.max_q and kv_len >= cfg.min_kv):
        return orig(q, k, v, scale=scale, mask=mask, sinks=sinks, **kw)
    is_str_mask = isinstance(mask, str)
    is_arr_mask = isinstance(mask, torch.Tensor)
    if is_arr_mask:
        mq = mask.shape[-2] if mask.dim() >= 2 else 1
        if mq not in (1, q_len):
            return orig(q, k, v, scale=scale, mask=mask, sinks=sinks, **kw)
    outs = []
    off = 0
    for p in _partition(q_len, cfg.max_chunk):
        qc = q[..., off:off + p, :]
        if mask is None:
            oc = orig(qc, k, v, scale=scale, mask=None, sinks=sinks, **kw)
        elif is_str_mask:
            end = kv_len - q_len + off + p
            oc = orig(qc, k[..., :end, :], v[..., :end, :], scale=scale, mask=mask, sinks=sinks, **kw)
        else:
            mc = mask if mask.shape[-2] == 1 else mask[..., off:off + p, :]
            oc = orig(qc, k, v, scale=scale, mask=mc, sinks=sinks, **kw)
        outs.append(oc)
        off += p
    return torch.cat(outs, dim=-2)


_ACTIVE: SplitConfig | None = None


def _patched_call(q, k, v, *, scale, mask=None, sinks=None, **kw):
    cfg = _ACTIVE
    if cfg is None:
        return _ORIG_SDPA(q, k, v, scale=scale, mask=mask, sinks=sinks, **kw)
    return split_sdpa(q, k, v, scale=scale, mask=mask, sinks=sinks, cfg=cfg, _orig=_ORIG_SDPA, **kw)


@contextlib.contextmanager
def sdpa_split(cfg: SplitConfig | None):
    """Route ``fast.scaled_dot_product_attention`` through the split while active. No-op when
    ``cfg`` is None or the split is already installed."""
    global _ACTIVE
    if cfg is None or fast.scaled_dot_product_attention is _patched_call:
        yield
        return
    prev = fast.scaled_dot_product_attention
    prev_cfg = _ACTIVE
    _ACTIVE = cfg
    fast.scaled_dot_product_attention = _patched_call
    try:
        yield
    finally:
        fast.scaled_dot_product_attention = prev
        _ACTIVE = prev_cfg


def patchable() -> bool:
    """True iff the attention entry point can be replaced (always, on this module)."""
    try:
        orig = fast.scaled_dot_product_attention
        fast.scaled_dot_product_attention = orig
        return True
    except (AttributeError, TypeError):
        return False
