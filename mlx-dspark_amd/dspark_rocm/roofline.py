"""Byte accounting of a decode / verify step: the denominators of every GB/s figure.

The reference's accounting rules (roofline.py:193-284), which ``weight_footprint`` and
``baseline_mbu`` keep so their numbers compare:

* a parameter under a routed-expert container (name containing ``.switch_mlp.``, the mlx-lm
  convention) is read for ``top_k / n_experts`` of its bytes per token; shared experts and every
  other tensor are read in full;
* the token embedding is a row gather, not a read of the table, so it does not count, unless
  the checkpoint has no separate ``lm_head`` (tied embeddings: the output head then reads the
  whole table);
* KV bytes grow with the context; model-bandwidth utilisation is bytes per step over the step
  time, against a bandwidth.

Below them sit the per-kernel algorithmic bytes of this build's hot path (qmm, verify
attention, MoE block), which bench.py quotes.
"""

from __future__ import annotations

_EXPERT_COUNT_KEYS = ("num_experts", "num_local_experts", "n_routed_experts")
_TOP_K_KEYS = ("num_experts_per_tok", "experts_per_token")


def _first_int(cfg: dict, keys) -> int | None:
    for key in keys:
        v = cfg.get(key)
        if v:
            return v if isinstance(v, int) else None
    return None


def _experts_from_config(cfg: dict | None) -> tuple[int | None, int | None]:
    """(routed experts, experts per token) from a HF-style config, looking inside
    ``text_config`` first (multimodal checkpoints) and then at the top level."""
    cfg = cfg or {}
    for scope in (cfg.get("text_config") or {}, cfg):
        n = _first_int(scope, _EXPERT_COUNT_KEYS)
        if n is not None and n > 1:
            k = _first_int(scope, _TOP_K_KEYS)
            return n, (k if k is not None and k > 0 else None)
    return None, None


def _kind(name: str) -> str:
    if ".switch_mlp." in name:
        return "expert"
    if ".embed_tokens." in name or name.endswith("embed_tokens.weight"):
        return "embed"
    return "dense"


def weight_footprint(params: list[tuple[str, int]], cfg: dict | None = None) -> dict:
    """Bytes one decode step reads, from ``[(param_name, nbytes), ...]``: ``total_bytes``
    (resident) and ``active_bytes`` (the roofline denominator), with the expert and embedding
    shares and whether the active figure is an estimate (experts present but no top-k known)."""
    by_kind = {"expert": 0, "embed": 0, "dense": 0}
    for name, nbytes in params:
        by_kind[_kind(name)] += int(nbytes or 0)
    tied = not any(name.endswith("lm_head.weight") for name, _ in params)
    n_experts, top_k = _experts_from_config(cfg)
    experts = by_kind["expert"]
    moe = bool(experts and n_experts)
    expert_share = top_k / n_experts if moe and top_k else 1.0
    active = by_kind["dense"] + int(experts * expert_share) + (by_kind["embed"] if tied else 0)
    return {
        "total_bytes": sum(by_kind.values()),
        "active_bytes": active,
        "expert_bytes": experts,
        "embed_bytes": by_kind["embed"],
        "is_moe": moe,
        "n_experts": n_experts if moe else None,
        "experts_per_tok": top_k if moe else None,
        "active_is_estimate": bool(experts) and not (moe and top_k),
    }


def bytes_per_token(active_bytes: int, kv_bytes_per_token: int | None, context: int) -> int:
    """Weights read once plus the KV of ``context`` earlier tokens."""
    return int(active_bytes) + int(kv_bytes_per_token or 0) * max(int(context or 0), 0)


def ceiling_tps(bandwidth_gb_s: float | None, bytes_per_tok: int) -> float | None:
    """Tokens per second if a step did nothing but read its bytes at this bandwidth."""
    return bandwidth_gb_s * 1e9 / bytes_per_tok if bandwidth_gb_s and bytes_per_tok > 0 else None


def roofline(*, bandwidth_gb_s: float | None, active_bytes: int, kv_bytes_per_token: int | None,
             context: int = 0) -> dict:
    """Bytes per token and the bandwidth ceiling at one context depth."""
    per_token = bytes_per_token(active_bytes, kv_bytes_per_token, context)
    return {"context": int(context or 0), "bytes_per_token": per_token,
            "ceiling_tps": ceiling_tps(bandwidth_gb_s, per_token)}


def baseline_mbu(step_ms: float | None, bytes_per_tok: int, bandwidth_gb_s: float | None) -> dict | None:
    """Model-bandwidth utilisation of a measured step: achieved GB/s and its fraction of
    ``bandwidth_gb_s`` (None when no bandwidth is given). None for a missing step time."""
    if not step_ms or step_ms <= 0 or bytes_per_tok <= 0:
        return None
    achieved = bytes_per_tok / (step_ms * 1e-3) / 1e9
    return {"step_ms": round(float(step_ms), 3), "achieved_gb_s": round(achieved, 1),
            "mbu": round(achieved / bandwidth_gb_s, 4) if bandwidth_gb_s else None}


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
