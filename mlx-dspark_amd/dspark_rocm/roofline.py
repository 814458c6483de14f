"""Byte accounting of a decode / verify step: the denominators of every GB/s figure.

Mirrors the reference's roofline.py:203-284 (``weight_footprint``, ``bytes_per_token``,
``ceiling_tps``, ``roofline``, ``baseline_mbu``): routed-expert tensors (names containing
``.switch_mlp.``, the mlx-lm convention) count ``top_k / n_experts`` of their bytes; the
embedding table is a row gather and is excluded unless there is no separate ``lm_head`` (tied
embeddings: the same table is then read in full by the output head). Also the per-kernel
algorithmic bytes of this build's hot path (qmm, verify attention, MoE block).
"""

from __future__ import annotations

_ROUTED_EXPERT_MARKERS = (".switch_mlp.",)


def _experts_from_config(cfg: dict | None) -> tuple[int | None, int | None]:
    cfg = cfg or {}
    for c in (cfg.get("text_config") or {}, cfg):
        n = c.get("num_experts") or c.get("num_local_experts") or c.get("n_routed_experts")
        k = c.get("num_experts_per_tok") or c.get("experts_per_token")
        if isinstance(n, int) and n > 1:
            return n, (k if isinstance(k, int) and k > 0 else None)
    return None, None


def weight_footprint(params: list[tuple[str, int]], cfg: dict | None = None) -> dict:
    """Bytes one decode step reads, from ``[(param_name, nbytes), ...]``: ``total_bytes``
    (resident) and ``active_bytes`` (the roofline denominator)."""
    names = [n for n, _ in params]
    has_lm_head = any(n.endswith("lm_head.weight") for n in names)
    n_experts, top_k = _experts_from_config(cfg)
    total = active = expert_bytes = embed_bytes = 0
    for name, nbytes in params:
        nbytes = int(nbytes or 0)
        total += nbytes
        if any(m in name for m in _ROUTED_EXPERT_MARKERS):
            expert_bytes += nbytes
            continue
        if ".embed_tokens." in name or name.endswith("embed_tokens.weight"):
            embed_bytes += nbytes
            continue
        active += nbytes
    is_moe = expert_bytes > 0 and bool(n_experts)
    if expert_bytes:
        frac = (top_k / n_experts) if (is_moe and top_k) else 1.0
        active += int(expert_bytes * frac)
    if not has_lm_head:
        active += embed_bytes
    return {
        "total_bytes": total,
        "active_bytes": active,
        "expert_bytes": expert_bytes,
        "embed_bytes": embed_bytes,
        "is_moe": is_moe,
        "n_experts": n_experts if is_moe else None,
        "experts_per_tok": top_k if is_moe else None,
        "active_is_estimate": bool(expert_bytes and not (is_moe and top_k)),
    }


def bytes_per_token(active_bytes: int, kv_bytes_per_token: int | None, context: int) -> int:
    return int(active_bytes) + int(kv_bytes_per_token or 0) * max(int(context or 0), 0)


def ceiling_tps(bandwidth_gb_s: float | None, bytes_per_tok: int) -> float | None:
    """Single-stream decode ceiling: one full weight (+KV) read per token at this bandwidth."""
    if not bandwidth_gb_s or bytes_per_tok <= 0:
        return None
    return bandwidth_gb_s * 1e9 / bytes_per_tok


def roofline(*, bandwidth_gb_s: float | None, active_bytes: int, kv_bytes_per_token: int | None,
             context: int = 0) -> dict:
    bpt = bytes_per_token(active_bytes, kv_bytes_per_token, context)
    return {"context": int(context or 0), "bytes_per_token": bpt, "ceiling_tps": ceiling_tps(bandwidth_gb_s, bpt)}


def baseline_mbu(step_ms: float | None, bytes_per_tok: int, bandwidth_gb_s: float | None) -> dict | None:
    """Model-bandwidth utilisation of a measured step: bytes / step against a bandwidth."""
    if not step_ms or step_ms <= 0 or bytes_per_tok <= 0:
        return None
    achieved = bytes_per_tok / (step_ms / 1e3) / 1e9
    out = {"step_ms": round(float(step_ms), 3), "achieved_gb_s": round(achieved, 1), "mbu": None}
    if bandwidth_gb_s:
        out["mbu"] = round(achieved / bandwidth_gb_s, 4)
    return out


# ---- algorithmic bytes of the hot-path kernels (HBM reads + writes that cannot be avoided)

def qmm_param_bytes(n: int, k: int, bits: int, group_size: int = 64) -> int:
    """Packed weights plus bf16 scales and biases of one [n, k] matrix."""
    return n * k * bits // 8 + 2 * 2 * n * (k // group_size)


def qmm_bytes(n: int, k: int, bits: int, m: int, group_size: int = 64) -> int:
    """One qmm launch: parameters + bf16 x [m, k] + bf16 y [m, n]."""
    return qmm_param_bytes(n, k, bits, group_size) + 2 * m * (k + n)


def attention_bytes(hq: int, hk: int, d: int, q_len: int, kv_len: int, batch: int = 1) -> int:
    """Verify attention: bf16 K and V of kv_len keys per KV head, q read and out written."""
    return batch * (2 * 2 * hk * kv_len * d + 2 * 2 * hq * q_len * d)


def moe_bytes(distinct_experts: int, h: int, i: int, bits: int, m: int, e: int, group_size: int = 64) -> int:
    """One routed-expert block: gate, up and down of each selected expert once, plus the bf16
    activations in, the logits and the output."""
    per = 2 * qmm_param_bytes(i, h, bits, group_size) + qmm_param_bytes(h, i, bits, group_size)
    return distinct_experts * per + 2 * m * h * 2 + 2 * m * e


def kv_bytes_per_token(layers: int, hk: int, d: int, elem_bytes: int = 2) -> int:
    """K and V of one token across the layers of a dense model."""
    return layers * 2 * hk * d * elem_bytes
