"""Dense verify forward of a qwen3-style 8-bit model, restated on the CPU (TEST INFRASTRUCTURE).

The reference's verify forward (target.py:642-677 -> run / _body_mlxlm / _head_mlxlm,
:187-221, :347-354) runs mlx-lm's decoder: embed -> per layer [RMSNorm -> q/k/v projections ->
per-head q/k RMSNorm -> RoPE at the cache offset -> cache write -> causal SDPA -> o projection
-> residual -> RMSNorm -> SwiGLU MLP -> residual] -> final RMSNorm -> lm_head. Every op's
result is bf16 (mlx op semantics); the rounding points restated here are:

    h  = bf16(x + r)
    rmsnorm(h, w) = bf16(bf16(h * rsqrt(mean(h^2) + eps)) * w)       (fp32 statistics)
    rope: pairs (i, i + D/2), angle = fp32(pos) * fp32(2^(-(2i/D) * log2(base))),
          y_i = bf16(x_i cos - x_{i+D/2} sin), y_{i+D/2} = bf16(x_i sin + x_{i+D/2} cos)
    swiglu(g, u) = bf16(bf16(g * bf16(sigmoid(g))) * u)
    projections: bf16 of the exact affine qmm (qmm_ref); attention: bf16 of the exact SDPA.

Pinned by tests/test_oracle_model.py: RMSNorm / RoPE closed forms (position 0 is the
identity, rotations preserve pair norms, scores depend only on relative position), a
float64 re-derivation of one layer, and the greedy accept / rollback KATs of verify_ref.
"""

from __future__ import annotations

import numpy as np

from .attn_ref import attention
from .moe_ref import swiglu
from .qmm_ref import qmm_f64
from .quant_ref import bf16_round


def bf(a) -> np.ndarray:
    return bf16_round(np.asarray(a, dtype=np.float32))


def rmsnorm(h, w, eps: float) -> np.ndarray:
    h = np.asarray(h, dtype=np.float32)
    inv = (1.0 / np.sqrt((h.astype(np.float64) ** 2).mean(axis=-1, keepdims=True) + eps)).astype(np.float32)
    return bf(bf(h * inv) * np.asarray(w, dtype=np.float32))


def rope(x, pos, base: float) -> np.ndarray:
    """x [..., L, D] bf16-valued, pos [L] absolute positions."""
    x = np.asarray(x, dtype=np.float32)
    D = x.shape[-1]
    half = D // 2
    i = np.arange(half, dtype=np.float32)
    inv_freq = np.exp2(-(2.0 * i / np.float32(D)) * np.float32(np.log2(np.float32(base)))).astype(np.float32)
    ang = (np.asarray(pos, dtype=np.float32)[:, None] * inv_freq[None, :]).astype(np.float32)
    c, s = np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))
    x1, x2 = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
    return np.concatenate([bf(x1 * c - x2 * s), bf(x1 * s + x2 * c)], axis=-1)


def qmm(x, lin) -> np.ndarray:
    w, s, b, bits = lin
    return bf(qmm_f64(np.asarray(x, dtype=np.float32), w, s, b, bits))


def qmm_c(x, lin) -> np.ndarray:
    """:func:`qmm` through the C restatement (dspark_oracle.c ``orc_qmm``, fp32 factored form,
    pinned to :func:`qmm_f64` by tests/test_oracle_qmm.py): for matrices too large for the
    float64 numpy path (a 151936-row vocabulary head, 25600-wide MLPs)."""
    from . import c_oracle
    from .quant_ref import bf16_bits

    w, s, b, bits = lin
    y = c_oracle.qmm(bf16_bits(np.asarray(x, np.float32)), w, bf16_bits(np.asarray(s, np.float32)),
                     bf16_bits(np.asarray(b, np.float32)), bits)
    return bf(y)


class DenseRef:
    """Weights as numpy: per layer dict of linears (packed uint32, scales, biases (fp32
    bf16-valued), bits) and norm weights; embed [V, H] fp32 (bf16-valued), or any object whose
    ``[ids]`` returns those rows. ``matmul`` evaluates one projection (default :func:`qmm`)."""

    def __init__(self, cfg: dict, embed, layers: list[dict], norm, lm_head, matmul=None, kv_bits=None):
        self.cfg, self.embed, self.layers, self.norm, self.lm_head = cfg, embed, layers, norm, lm_head
        self.matmul = matmul or qmm
        self.kv_bits = kv_bits      # quantized caches (target.py:166-184): rows kept as scale * q + bias
        c = cfg
        self.k = [np.zeros((c["kv_heads"], 0, c["head_dim"]), np.float32) for _ in layers]
        self.v = [np.zeros((c["kv_heads"], 0, c["head_dim"]), np.float32) for _ in layers]
        self.offset = 0

    def seed_cache(self, keys: list, values: list) -> None:
        """Start from caches already holding ``keys[l]`` / ``values[l]`` [Hk, L, D] per layer
        (bf16-valued), e.g. a synthetic prefix; the offset becomes L."""
        self.k = [np.asarray(k, np.float32) for k in keys]
        self.v = [np.asarray(v, np.float32) for v in values]
        self.offset = self.k[0].shape[1]

    def forward(self, ids, tap=None) -> np.ndarray:
        """ids [M] at positions offset..offset+M-1 -> logits [M, V]; appends to the caches.
        With ``tap`` (layer indices), ``self.fused`` [M, n_tap * H] holds the residual stream
        after each tapped layer, in layer order (target.py:208-220 ``_body_mlxlm``)."""
        c = self.cfg
        tapset = {int(i) for i in tap} if tap is not None else set()
        captured = []
        M = len(ids)
        Hq, Hk, D, eps = c["heads"], c["kv_heads"], c["head_dim"], c["eps"]
        pos = np.arange(self.offset, self.offset + M)
        h = np.asarray(self.embed[np.asarray(ids)], np.float32)
        qmm = self.matmul
        r = None
        for li, L in enumerate(self.layers):
            if r is not None:
                h = bf(h + r)
                if li - 1 in tapset:
                    captured.append(h)
            y = rmsnorm(h, L["input_norm"], eps)
            q = qmm(y, L["q"]).reshape(M, Hq, D).transpose(1, 0, 2)
            k = qmm(y, L["k"]).reshape(M, Hk, D).transpose(1, 0, 2)
            v = qmm(y, L["v"]).reshape(M, Hk, D).transpose(1, 0, 2)
            q = rope(rmsnorm(q, L["q_norm"], eps), pos, c["rope_theta"])
            k = rope(rmsnorm(k, L["k_norm"], eps), pos, c["rope_theta"])
            if self.kv_bits:
                k, v = self._kv_quantized(k), self._kv_quantized(v)
            self.k[li] = np.concatenate([self.k[li][:, :self.offset], k], axis=1)
            self.v[li] = np.concatenate([self.v[li][:, :self.offset], v], axis=1)
            att = bf(attention(q[None], self.k[li][None], self.v[li][None], D ** -0.5, causal=True)[0])
            o = qmm(att.transpose(1, 0, 2).reshape(M, Hq * D), L["o"])
            h = bf(h + o)
            y2 = rmsnorm(h, L["post_norm"], eps)
            r = qmm(swiglu(qmm(y2, L["gate"]), qmm(y2, L["up"])), L["down"])
        h = bf(h + r)
        if len(self.layers) - 1 in tapset:
            captured.append(h)
        self.fused = np.concatenate(captured, axis=-1) if captured else np.zeros((M, 0), np.float32)
        self.offset += M
        return qmm(rmsnorm(h, self.norm, eps), self.lm_head)

    def _kv_quantized(self, x) -> np.ndarray:
        """Rows [Hk, M, D] as a quantized cache holds them: quantized in groups of 64 along D
        with quant_ref's rule, dequantized exactly (float64)."""
        from .quant_ref import dequantize, quantize

        hk, m, d = x.shape
        w, s, b = quantize(np.asarray(x, np.float32).reshape(hk * m, d), self.kv_bits)
        return dequantize(w, s, b, self.kv_bits).reshape(hk, m, d)

    def trim(self, n: int) -> None:
        n = min(self.offset, max(0, int(n)))
        self.offset -= n
