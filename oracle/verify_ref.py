"""Greedy accept and dense KV rollback, restated from the reference decode loop.

* accept (generate.py:1544-1555): tt = argmax(verify logits); n = sum(cumprod(draft == tt[:len(draft)]));
  committed = draft[:n] + [tt[n]] (the accepted prefix plus the target's bonus token).
* rollback (target.py:679-696): dense targets trim every KV cache by len(draft) - n; 0 is a no-op.
* trim (batch_engine.py:220-224): metadata only, offset -= n clamped at 0; the next write overwrites.
* bookkeeping (generate.py:1590-1593, :111-113): n_cached += n + 1; mean_accept_len =
  num_tokens / num_rounds.

Pinned by the reference tests' own cases (tests/test_bonsai.py:399-415,
tests/test_batch_engine.py:57-73) restated as KATs in tests/test_oracle_verify.py.
"""

from __future__ import annotations

import numpy as np


def greedy_accept(draft: list[int], tt: list[int]) -> tuple[int, list[int]]:
    n = 0
    for d, t in zip(draft, tt):
        if d != t:
            break
        n += 1
    return n, list(draft[:n]) + [int(tt[n])]


class KVCacheRef:
    """[H, cap, D] buffer with an offset (one layer, batch 1)."""

    def __init__(self, heads: int, cap: int, dim: int, dtype=np.float32):
        self.k = np.zeros((heads, cap, dim), dtype=dtype)
        self.v = np.zeros((heads, cap, dim), dtype=dtype)
        self.offset = 0

    def update_and_fetch(self, k: np.ndarray, v: np.ndarray):
        t = k.shape[1]
        self.k[:, self.offset:self.offset + t] = k
        self.v[:, self.offset:self.offset + t] = v
        self.offset += t
        return self.k[:, :self.offset], self.v[:, :self.offset]

    def trim(self, n: int) -> int:
        n = min(self.offset, max(0, int(n)))
        self.offset -= n
        return n


def rollback(caches, n_rejected: int) -> None:
    if n_rejected > 0:
        for c in caches:
            c.trim(n_rejected)


def mean_accept_len(num_tokens: int, num_rounds: int) -> float:
    return num_tokens / max(num_rounds, 1)
