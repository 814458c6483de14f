"""``scaled_dot_product_attention`` with MLX's calling convention: the patchable attention
entry point of the verify forward (the role ``mx.fast.scaled_dot_product_attention`` plays in
the reference; multirow_attn.py:50 and sdpa_split.py:38 capture and replace it).

Callers look the function up on this module at call time (``fast.scaled_dot_product_attention``)
so the scopes in :mod:`.sdpa_split` and :mod:`.multirow_attn` can route it. The function
defined here is the stock path: fp32 scores and softmax, output in q's dtype, computed with
torch ops on q's device.

Semantics (MLX's): q [B, Hq, qL, D], k/v [B, Hk, L, D] with Hq % Hk == 0 (GQA: query head h
reads KV head h // (Hq/Hk)). ``mask`` is None, the string "causal" (row i sees keys
0 .. L - qL + i, bottom-right aligned), a boolean array (True = visible) or an additive
array, broadcastable to [B, Hq, qL, L]. ``sinks`` (optional [Hq]) adds one logit per head to
every row's softmax normaliser without a value.
"""

from __future__ import annotations

import torch


def _expand_kv(t: torch.Tensor, hq: int) -> torch.Tensor:
    hk = t.shape[1]
    if hk == hq:
        return t
    return t.repeat_interleave(hq // hk, dim=1)


def causal_mask(q_len: int, kv_len: int, device=None) -> torch.Tensor:
    """Boolean [q_len, kv_len]: row i sees keys 0 .. kv_len - q_len + i."""
    i = torch.arange(q_len, device=device).unsqueeze(1)
    j = torch.arange(kv_len, device=device).unsqueeze(0)
    return j <= (kv_len - q_len + i)


def _stock_sdpa(q, k, v, *, scale, mask=None, sinks=None):
    B, Hq, qL, D = q.shape
    L = k.shape[2]
    if k.shape[1] == 0 or Hq % k.shape[1]:
        raise ValueError(f"Hq={Hq} is not a multiple of Hk={k.shape[1]}")
    kk = _expand_kv(k, Hq).to(torch.float32)
    vv = _expand_kv(v, Hq).to(torch.float32)
    s = torch.matmul(q.to(torch.float32), kk.transpose(-1, -2).contiguous()) * float(scale)
    if isinstance(mask, str):
        if mask != "causal":
            raise ValueError(f"mask={mask!r}: only 'causal' is a string mask")
        s = s.masked_fill(~causal_mask(qL, L, q.device), float("-inf"))
    elif mask is not None:
        if mask.dtype == torch.bool:
            s = s.masked_fill(~mask, float("-inf"))
        else:
            s = s + mask.to(torch.float32)
    if sinks is not None:
        sk = sinks.to(torch.float32).reshape(1, Hq, 1, 1).expand(B, Hq, qL, 1)
        s = torch.cat([s, sk], dim=-1)
        p = torch.softmax(s, dim=-1)[..., :L]
    else:
        p = torch.softmax(s, dim=-1)
    return torch.matmul(p, vv).to(q.dtype)


def scaled_dot_product_attention(q, k, v, *, scale, mask=None, sinks=None, **kw):
    if kw:
        raise TypeError(f"unexpected arguments {sorted(kw)}")
    return _stock_sdpa(q, k, v, scale=scale, mask=mask, sinks=sinks)


STOCK = scaled_dot_product_attention


def quantized_scaled_dot_product_attention(q, q_keys, q_values, *, scale, mask=None, group_size: int = 64,
                                           bits: int = 8):
    """Attention over quantized K/V triples (words, scales, biases), the helper mlx-lm's
    attention layers call when their cache has ``bits``: the stock path dequantizes
    (``scale * field + bias`` in fp32) and runs :func:`scaled_dot_product_attention` in fp32,
    output in q's dtype. Patchable like the plain entry point."""
    from .quant import unpack

    def deq(trip):
        w, s, b = trip
        lead = w.shape[:-1]
        vals = unpack(w.reshape(-1, w.shape[-1]), bits).to(torch.float32).reshape(*lead, -1)
        g = vals.reshape(*lead, -1, group_size)
        return (g * s.to(torch.float32).unsqueeze(-1) + b.to(torch.float32).unsqueeze(-1)).reshape(*lead, -1)

    return _stock_sdpa(q.to(torch.float32), deq(q_keys), deq(q_values), scale=scale, mask=mask).to(q.dtype)


QUANTIZED_STOCK = quantized_scaled_dot_product_attention
