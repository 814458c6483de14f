"""Scoped replacement of a module or class attribute, shared by the three dispatch scopes
(``small_m_matmul``, ``multirow_attention``, ``sdpa_split``).

A scope swaps one attribute for the duration of a ``with`` block and puts back exactly the
object it found on entry, so scopes stack in any order and another scope that replaced the same
attribute in between is restored to, not overwritten (the reference's patches behave this way:
small_m_qmm.py:83-106, multirow_attn.py:338-370, sdpa_split.py:106-124). Each scope's
configuration lives in a :class:`Slot` whose value is restored the same way.
"""

from __future__ import annotations

import contextlib
from typing import Any, Iterator


class Slot:
    """One value a scope sets while active (its allowlist, window config, tree mask ...)."""

    __slots__ = ("value",)

    def __init__(self, value: Any = None):
        self.value = value

    @contextlib.contextmanager
    def holding(self, value: Any) -> Iterator[None]:
        saved, self.value = self.value, value
        try:
            yield
        finally:
            self.value = saved


@contextlib.contextmanager
def replaced(owner: Any, name: str, new: Any) -> Iterator[Any]:
    """``owner.name = new`` inside the block; yields the object found on entry, which is put
    back on exit (also on an exception)."""
    found = getattr(owner, name)
    setattr(owner, name, new)
    try:
        yield found
    finally:
        setattr(owner, name, found)


def can_replace(owner: Any, name: str) -> bool:
    """Whether ``owner.name`` accepts assignment (set to itself; nothing changes)."""
    try:
        setattr(owner, name, getattr(owner, name))
    except (AttributeError, TypeError):
        return False
    return True
