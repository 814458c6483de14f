"""bf16 KV cache with O(1) rollback, laid out for the verify-attention kernel.

Semantics follow the caches the reference drives (mlx-lm ``KVCache``; its own ``BatchCache``,
batch_engine.py:193-224): buffers ``[B, Hk, capacity, D]`` grown in steps of :data:`STEP` rows
(batch_engine.py:38, :226-227); :meth:`update_and_fetch` writes T rows at ``offset`` and returns
``[..., :offset, :]`` views (no copy — the kernel reads the strides); :meth:`trim` is pure
metadata: ``offset -= n`` clamped at 0, the next write overwrites the stale tail
(batch_engine.py:220-224; tests/test_batch_engine.py:57-73). Dense rollback trims every layer's
cache by the rejected count (target.py:679-696).

MI355X layout note: with 288 GB of HBM the cache is allocated once at its final capacity when
the caller knows it (``capacity=``), so verify rounds never reallocate; growth copies only when
an unknown length overflows.
"""

from __future__ import annotations

import torch

STEP = 256


def _round_step(n: int) -> int:
    return ((n + STEP - 1) // STEP) * STEP


class KVCache:
    def __init__(self, batch: int, kv_heads: int, head_dim: int, *, device, capacity: int = 0,
                 dtype=torch.bfloat16):
        self.batch, self.kv_heads, self.head_dim = batch, kv_heads, head_dim
        self.device, self.dtype = torch.device(device), dtype
        cap = _round_step(max(capacity, 1))
        self.keys = torch.zeros((batch, kv_heads, cap, head_dim), dtype=dtype, device=self.device)
        self.values = torch.zeros_like(self.keys)
        self.offset = 0

    @property
    def capacity(self) -> int:
        return self.keys.shape[2]

    def _grow(self, need: int) -> None:
        cap = _round_step(need)
        nk = torch.zeros((self.batch, self.kv_heads, cap, self.head_dim), dtype=self.dtype, device=self.device)
        nv = torch.zeros_like(nk)
        nk[:, :, :self.offset] = self.keys[:, :, :self.offset]
        nv[:, :, :self.offset] = self.values[:, :, :self.offset]
        self.keys, self.values = nk, nv

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Write ``keys``/``values`` [B, Hk, T, D] at ``offset``; return the ``[..., :offset, :]`` views."""
        t = keys.shape[2]
        if self.offset + t > self.capacity:
            self._grow(self.offset + t)
        self.keys[:, :, self.offset:self.offset + t] = keys
        self.values[:, :, self.offset:self.offset + t] = values
        self.offset += t
        return self.fetch()

    def reserve(self, t: int) -> None:
        """Make room for ``t`` more rows at ``offset`` (a kernel then writes them in place)."""
        if self.offset + t > self.capacity:
            self._grow(self.offset + t)

    def advance(self, t: int) -> None:
        """Commit ``t`` rows a kernel wrote at ``offset`` (after :meth:`reserve`)."""
        if self.offset + t > self.capacity:
            raise ValueError(f"advance({t}) past capacity {self.capacity} at offset {self.offset}")
        self.offset += t

    def fetch(self):
        return self.keys[:, :, :self.offset, :], self.values[:, :, :self.offset, :]

    def trim(self, n: int) -> int:
        """Roll back ``n`` rows (metadata only). Returns how many were removed."""
        n = min(self.offset, max(0, int(n)))
        self.offset -= n
        return n

    def is_trimmable(self) -> bool:
        return True

    @property
    def state(self):
        return self.fetch()


class QuantizedKVCache:
    """KV cache holding affine-quantized rows: mlx-lm's ``QuantizedKVCache`` layout, which the
    reference's targets use when ``kv_bits`` is set (target.py:166-184). Keys and values are
    each ``(words int32 [B, Hk, cap, D*bits/32], scales [B, Hk, cap, D/64], biases ...)`` with
    scales and biases in the model dtype; rows are quantized as they are written
    (:func:`dspark_rocm.quant.quantize_rows`). Offset, ``trim`` and growth behave as in
    :class:`KVCache`; :meth:`update_and_fetch` returns the two triples as ``[..., :offset, :]``
    views, which ``ops.verify_attention_quantized`` reads in place."""

    def __init__(self, batch: int, kv_heads: int, head_dim: int, *, bits: int = 8, group_size: int = 64, device,
                 capacity: int = 0, dtype=torch.bfloat16):
        self.batch, self.kv_heads, self.head_dim = batch, kv_heads, head_dim
        self.bits, self.group_size = bits, group_size
        self.device, self.dtype = torch.device(device), dtype
        self.keys = self._alloc(_round_step(max(capacity, 1)))
        self.values = self._alloc(self.keys[0].shape[2])
        self.offset = 0

    def _alloc(self, cap: int):
        B, H, D = self.batch, self.kv_heads, self.head_dim
        w = torch.zeros((B, H, cap, D * self.bits // 32), dtype=torch.int32, device=self.device)
        s = torch.zeros((B, H, cap, D // self.group_size), dtype=self.dtype, device=self.device)
        return (w, s, torch.zeros_like(s))

    @property
    def capacity(self) -> int:
        return self.keys[0].shape[2]

    def _grow(self, need: int) -> None:
        cap = _round_step(need)
        nk, nv = self._alloc(cap), self._alloc(cap)
        for new, old in zip(nk + nv, self.keys + self.values):
            new[:, :, :self.offset] = old[:, :, :self.offset]
        self.keys, self.values = nk, nv

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        """Quantize ``keys``/``values`` [B, Hk, T, D] into rows ``offset..offset+T``; return the
        ``[..., :offset, :]`` views of both triples."""
        from .quant import quantize_rows

        t = keys.shape[2]
        if self.offset + t > self.capacity:
            self._grow(self.offset + t)
        for dst, src in ((self.keys, keys), (self.values, values)):
            for buf, part in zip(dst, quantize_rows(src, self.bits, self.group_size, self.dtype)):
                buf[:, :, self.offset:self.offset + t] = part
        self.offset += t
        return self.fetch()

    def reserve(self, t: int) -> None:
        """Make room for ``t`` more rows at ``offset`` (a kernel then writes them in place)."""
        if self.offset + t > self.capacity:
            self._grow(self.offset + t)

    def advance(self, t: int) -> None:
        """Commit ``t`` rows a kernel wrote at ``offset`` (after :meth:`reserve`)."""
        if self.offset + t > self.capacity:
            raise ValueError(f"advance({t}) past capacity {self.capacity} at offset {self.offset}")
        self.offset += t

    def fetch(self):
        view = lambda trip: tuple(a[:, :, :self.offset] for a in trip)
        return view(self.keys), view(self.values)

    def trim(self, n: int) -> int:
        n = min(self.offset, max(0, int(n)))
        self.offset -= n
        return n

    def is_trimmable(self) -> bool:
        return True

    @property
    def state(self):
        return self.fetch()
