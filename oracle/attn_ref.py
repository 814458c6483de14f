"""Causal-in-block GQA verify attention, restated from the reference.

Definitions (multirow_attn.py:52-178, :223-259; sdpa_split.py:61-93; A.2):

* q [B, Hq, Mq, D]; K/V [B, Hk, L, D] hold L keys including the Mq new rows.
* GQA: query head h reads KV head h // (Hq // Hk).
* causal: row i sees keys 0 .. L - Mq + i (bottom-right aligned, mlx's "causal");
* tree: keys < L - Mq always; key L - Mq + j iff bit j of anc[i] (multirow_attn.py:184-195).
* out = softmax(scale * q k^T + mask) v.

:func:`attention` evaluates that definition in float64 (the reference tests compare the kernel
against an fp32 SDPA, tests/test_multirow_attn.py:41-45). :func:`attention_multirow` restates the
multirow kernel's arithmetic: rows packed per KV head (row r = g*Mq + i), 16-key tiles, exp2
softmax with m initialised to -1e30, P rounded to bf16 before P.V, fp32 partials per key block,
then the 2^(m_j - M) combine (multirow_attn.py:86-177). :func:`split_sdpa` restates the row
split (sdpa_split.py:61-93).

Pinned by (tests/test_oracle_attn.py): a pure-Python per-element loop on tiny shapes; GQA equal
to MHA over tiled K/V; row independence (each row equals a 1-row call over its visible prefix);
the causal leak KAT (tests/test_multirow_attn.py:90-99); uniform keys -> mean of V; invariance of
the multirow restatement to its block split; agreement of the two forms within bf16 rounding.
"""

from __future__ import annotations

import math

import numpy as np

from .quant_ref import bf16_round

LOG2E = 1.4426950408889634


def visible_mask(mq: int, L: int, causal: bool = True, tree_anc=None) -> np.ndarray:
    """bool [Mq, L]: True where row i may attend key j."""
    j = np.arange(L)[None, :]
    i = np.arange(mq)[:, None]
    tail0 = L - mq
    if tree_anc is not None:
        anc = np.asarray(tree_anc, dtype=np.uint64)[:, None]
        rel = np.clip(j - tail0, 0, 63).astype(np.uint64)
        bit = ((anc >> rel) & np.uint64(1)).astype(bool)
        return (j < tail0) | bit
    if not causal:
        return np.ones((mq, L), dtype=bool)
    return j <= tail0 + i


def attention(q, k, v, scale: float, causal: bool = True, tree_anc=None, mask=None) -> np.ndarray:
    """float64 reference. ``mask`` (bool [Mq, L]) overrides causal/tree when given."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, mq, D = q.shape
    Hk, L = k.shape[1], k.shape[2]
    gqa = Hq // Hk
    vis = visible_mask(mq, L, causal, tree_anc) if mask is None else np.asarray(mask, dtype=bool)
    out = np.empty((B, Hq, mq, v.shape[-1]), dtype=np.float64)
    for b in range(B):
        for h in range(Hq):
            s = (q[b, h] @ k[b, h // gqa].T) * scale
            s = np.where(vis, s, -np.inf)
            s = s - s.max(axis=-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=-1, keepdims=True)
            out[b, h] = p @ v[b, h // gqa]
    return out


def plan_blocks(L: int, chunk: int) -> list[tuple[int, int]]:
    return [(k0, min(L, k0 + chunk)) for k0 in range(0, L, chunk)]


def attention_multirow(q, k, v, scale: float, causal: bool = True, tree_anc=None,
                       chunk: int | None = None, tile: int = 16) -> np.ndarray:
    """The multirow kernel's arithmetic in fp32 (bf16-valued inputs), output bf16-valued fp32."""
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    B, Hq, mq, D = q.shape
    Hk, L = k.shape[1], k.shape[2]
    gqa = Hq // Hk
    R = gqa * mq
    chunk = chunk or L
    vis = visible_mask(mq, L, causal, tree_anc)
    rows_vis = np.tile(vis, (gqa, 1))                 # row r = g*mq + i -> vis[i]
    sc = np.float32(scale * LOG2E)
    out = np.empty_like(q)
    for b in range(B):
        for hk in range(Hk):
            qq = q[b, hk * gqa:(hk + 1) * gqa].reshape(R, D)
            parts = []
            for k0, k1 in plan_blocks(L, chunk):
                m = np.full(R, -1e30, dtype=np.float32)
                l = np.zeros(R, dtype=np.float32)
                o = np.zeros((R, D), dtype=np.float32)
                for kt in range(k0, k1, tile):
                    ke = min(k1, kt + tile)
                    s = (qq @ k[b, hk, kt:ke].T).astype(np.float32)
                    s = np.where(rows_vis[:, kt:ke], s * sc, -np.inf).astype(np.float32)
                    mn = np.maximum(m, s.max(axis=1))
                    f = np.exp2(m - mn).astype(np.float32)
                    p = np.exp2(s - mn[:, None]).astype(np.float32)
                    l = (l * f + p.sum(axis=1)).astype(np.float32)
                    o = (o * f[:, None] + bf16_round(p) @ v[b, hk, kt:ke]).astype(np.float32)
                    m = mn
                parts.append((m, l, o))
            M = np.max(np.stack([pm for pm, _, _ in parts]), axis=0)
            num = np.zeros((R, D), dtype=np.float32)
            den = np.zeros(R, dtype=np.float32)
            for pm, pl, po in parts:
                w = np.exp2(pm - M).astype(np.float32)
                den += w * pl
                num += w[:, None] * po
            out[b, hk * gqa:(hk + 1) * gqa] = (num / den[:, None]).reshape(gqa, mq, D)
    return bf16_round(out)


def partition(q_len: int, max_chunk: int) -> list[int]:
    """Balanced split into ceil(q_len/max_chunk) chunks, larger first (sdpa_split.py:52-58)."""
    n = max(1, math.ceil(q_len / max_chunk))
    base, rem = divmod(q_len, n)
    return [base + 1] * rem + [base] * (n - rem)


def split_sdpa(q, k, v, scale: float, causal: bool, max_chunk: int) -> np.ndarray:
    """Row split with per-chunk causal K/V slicing (sdpa_split.py:78-93), float64."""
    mq, L = q.shape[2], k.shape[2]
    outs, off = [], 0
    for p in partition(mq, max_chunk):
        qc = q[:, :, off:off + p]
        if causal:
            end = L - mq + off + p
            outs.append(attention(qc, k[:, :, :end], v[:, :, :end], scale, causal=True))
        else:
            outs.append(attention(qc, k, v, scale, causal=False))
        off += p
    return np.concatenate(outs, axis=2)


def dequantize_kv(words, scales, biases, bits: int) -> np.ndarray:
    """Quantized cache rows (mlx-lm QuantizedKVCache: uint32 words [..., L, D*bits/32] of
    ``bits``-wide fields along D, low bits first; scales/biases [..., L, D/64]) -> float64
    [..., L, D] = scale * field + bias per group of 64 (the affine format of quant_ref)."""
    from .quant_ref import dequantize

    w = np.asarray(words).view(np.uint32)
    lead = w.shape[:-1]
    flat = dequantize(w.reshape(-1, w.shape[-1]), np.asarray(scales, np.float64).reshape(-1, scales.shape[-1]),
                      np.asarray(biases, np.float64).reshape(-1, biases.shape[-1]), bits)
    return flat.reshape(*lead, -1)


def attention_quantized(q, keys, values, scale: float, bits: int, causal: bool = True) -> np.ndarray:
    """float64 attention over dequantized K/V triples (words, scales, biases): the function the
    quantized-KV attention computes (dequantize, then the definition of :func:`attention`)."""
    return attention(q, dequantize_kv(*keys, bits), dequantize_kv(*values, bits), scale, causal=causal)
