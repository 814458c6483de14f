"""Pins oracle/verify_ref.py with the reference's own cases restated as KATs: greedy accept
(generate.py:1544-1555: n = sum(cumprod(draft == tt[:len(draft)])), committed = draft[:n] +
[tt[n]]), per-row trim and clamp (tests/test_batch_engine.py:57-73), dense rollback
(tests/test_bonsai.py:399-415), and mean_accept_len (generate.py:111-113)."""

from __future__ import annotations

import numpy as np

from oracle import verify_ref


def _cumprod_form(draft, tt):
    match = (np.asarray(draft) == np.asarray(tt[:len(draft)])).astype(np.int32)
    n = int(np.cumprod(match).sum()) if len(draft) else 0
    return n, list(draft[:n]) + [int(tt[n])]


def test_greedy_accept_kats():
    assert verify_ref.greedy_accept([5, 6, 7], [5, 6, 9, 1]) == (2, [5, 6, 9])
    assert verify_ref.greedy_accept([1, 2], [1, 2, 3]) == (2, [1, 2, 3])     # all accepted + bonus
    assert verify_ref.greedy_accept([4], [5, 6]) == (0, [5])                 # first token rejected
    assert verify_ref.greedy_accept([], [8]) == (0, [8])                     # no draft: plain decode
    assert verify_ref.greedy_accept([3, 9, 3], [3, 1, 3, 4]) == (1, [3, 1])  # a later match counts nothing


def test_greedy_accept_equals_reference_expression():
    r = np.random.Generator(np.random.PCG64(0))
    for _ in range(500):
        n = int(r.integers(0, 16))
        draft = r.integers(0, 4, n).tolist()
        tt = r.integers(0, 4, n + 1).tolist()
        assert verify_ref.greedy_accept(draft, tt) == _cumprod_form(draft, tt)


def test_trim_is_metadata_and_next_write_overwrites():
    c = verify_ref.KVCacheRef(2, 16, 4)
    c.update_and_fetch(np.ones((2, 5, 4)), np.ones((2, 5, 4)))
    assert c.offset == 5
    assert c.trim(2) == 2 and c.offset == 3
    k2 = np.full((2, 1, 4), 7.0)
    k, _ = c.update_and_fetch(k2, k2)
    assert c.offset == 4 and k.shape == (2, 4, 4) and np.all(k[:, 3] == 7.0) and np.all(k[:, :3] == 1.0)


def test_trim_clamps_at_zero():
    c = verify_ref.KVCacheRef(1, 8, 2)
    c.update_and_fetch(np.ones((1, 2, 2)), np.ones((1, 2, 2)))
    assert c.trim(5) == 2 and c.offset == 0
    assert c.trim(0) == 0 and c.offset == 0


def test_dense_rollback_trims_every_cache_and_zero_is_noop():
    caches = [verify_ref.KVCacheRef(1, 32, 2) for _ in range(2)]
    for c in caches:
        c.update_and_fetch(np.ones((1, 10, 2)), np.ones((1, 10, 2)))
    verify_ref.rollback(caches, 3)
    assert [c.offset for c in caches] == [7, 7]
    verify_ref.rollback(caches, 0)
    assert [c.offset for c in caches] == [7, 7]


def test_mean_accept_len():
    assert verify_ref.mean_accept_len(12, 4) == 3.0
    assert verify_ref.mean_accept_len(0, 0) == 0.0
