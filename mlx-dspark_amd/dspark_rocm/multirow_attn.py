"""Multi-row verify attention: the gfx950 kernel behind the reference's ``multirow_sdpa`` and
its scoped patch of the attention entry point.

Same API as the reference module (multirow_attn.py:204-488): ``plan``, ``multirow_sdpa``,
``Window``, ``MultirowConfig``, ``eligible``, ``tree_mask``, ``multirow_attention``,
``active`` and ``measure_window``. The kernel is ``dspark_verify_attention`` (split-KV pass
plus combine, v_mfma_f32_16x16x32_bf16); it serves bf16, head_dim 64 or 128, whole GQA groups
with gqa * q_len <= 256, and reads K/V through their batch/head/sequence strides (KV-cache
views sliced along the sequence axis are used in place).

``multirow_attention(cfg)`` patches :func:`dspark_rocm.fast.scaled_dot_product_attention`:
an eligible call of a measured shape (its :class:`Window`) runs the kernel — causal iff the
mask is the string "causal" and q_len > 1 — and every other call falls through to whatever
was installed before (the split scope, then the stock path) (multirow_attn.py:338-370). A
tree verify registers its exact mask object with :func:`tree_mask`; calls carrying that
object take the kernel's ancestry variant (multirow_attn.py:322-349).
"""

from __future__ import annotations

import contextlib
import ctypes
import math
from dataclasses import dataclass

import torch

from . import _lib, fast, ops

_ORIG_SDPA = fast.STOCK

MAX_D = 128
HEAD_DIMS = ops.ATTN_HEAD_DIMS
MAX_ROWS = 256          # gqa * q_len the kernel's row tiles cover
_DTYPES = (torch.bfloat16,)


def plan(hq: int, hk: int, q_len: int, d: int, kv_len: int, batch: int = 1) -> dict:
    """Launch geometry of the kernel for this shape (host query): rows R, padded rows RP, row
    groups NRG, keys per block CHUNK, key blocks NB and pass-1 workgroups."""
    out = (ctypes.c_int32 * 6)()
    _lib.check("dspark_verify_attention_plan",
               _lib.load().dspark_verify_attention_plan(batch, hq, hk, q_len, d, kv_len, out))
    return {"R": out[0], "RP": out[1], "NRG": out[2], "CHUNK": out[3], "NB": out[4], "workgroups": out[5]}


def multirow_sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float, causal: bool,
                  tree_anc: torch.Tensor | None = None) -> torch.Tensor:
    """``scaled_dot_product_attention(q, k, v, scale, mask="causal" if causal else None)`` for
    the few-row shapes (see :func:`eligible`); ``k``/``v`` may be strided cache views.
    ``tree_anc`` (uint32/int32 [q_len]): tree-verify visibility bits over the last q_len keys
    instead of the causal rule."""
    if tree_anc is not None:
        causal = False
    return ops.verify_attention(q, k, v, scale=scale, causal=causal, tree_anc=tree_anc)


@dataclass(frozen=True)
class Window:
    """Measured gate for one attention shape ``(hq, hk, d)``: the kernel serves calls with
    ``min_q <= q_len <= max_q`` and ``kv_len >= min_kv``."""
    hq: int
    hk: int
    d: int
    min_q: int = 2
    max_q: int = 16
    min_kv: int = 1024


@dataclass(frozen=True)
class MultirowConfig:
    """One :class:`Window` per measured attention shape; unmeasured shapes pass through."""
    windows: tuple[Window, ...] = ()

    def window(self, hq: int, hk: int, d: int) -> Window | None:
        for w in self.windows:
            if w.hq == hq and w.hk == hk and w.d == d:
                return w
        return None


def eligible(q, k, v, mask, sinks, cfg: MultirowConfig) -> bool:
    """Structural + gate check (multirow_attn.py:288-312), on GPU tensors."""
    return eligible_shape(q, k, v, mask, sinks, cfg) and q.is_cuda and k.is_cuda and v.is_cuda


def eligible_shape(q, k, v, mask, sinks, cfg: MultirowConfig) -> bool:
    """No sinks; mask None or "causal"; 4-D bf16 tensors of a measured shape; K/V/Q head dims
    equal and supported; whole GQA groups; q_len and the KV length inside the shape's window;
    K/V contiguous along head_dim (checked here — torch exposes strides)."""
    if sinks is not None or q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        return False
    if not (mask is None or (isinstance(mask, str) and mask == "causal")):
        return False
    B, Hq, qL, D = q.shape
    Hk, L = k.shape[1], k.shape[2]
    w = cfg.window(Hq, Hk, D)
    if w is None or not (w.min_q <= qL <= w.max_q and qL <= L) or max(w.min_kv, 16) > L:
        return False
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        return False
    if k.shape[-1] != D or v.shape[-1] != D or D not in HEAD_DIMS or v.shape[2] != L:
        return False
    if Hk == 0 or Hq % Hk or v.shape[1] != Hk or k.shape[0] != B or v.shape[0] != B:
        return False
    return not ((Hq // Hk) * qL > MAX_ROWS or k.stride(-1) != 1 or v.stride(-1) != 1)


_ACTIVE: MultirowConfig | None = None
_PREV = None
_TREE: tuple | None = None


@contextlib.contextmanager
def tree_mask(mask, anc_bits: torch.Tensor):
    """Declare ``mask`` (the exact object a tree verify passes) as a tree-verify mask whose
    visibility over the last W keys is ``anc_bits`` (uint32 per row). Identity-matched."""
    global _TREE
    prev = _TREE
    _TREE = (mask, anc_bits)
    try:
        yield
    finally:
        _TREE = prev


def _patched_call(q, k, v, *, scale, mask=None, sinks=None, **kw):
    cfg = _ACTIVE
    if cfg is not None and not kw:
        tree = _TREE
        if (tree is not None and mask is tree[0] and q.dim() == 4 and q.shape[2] <= 32
                and eligible(q, k, v, None, sinks, cfg)):
            return multirow_sdpa(q, k, v, scale=scale, causal=False, tree_anc=tree[1])
        if eligible(q, k, v, mask, sinks, cfg):
            return multirow_sdpa(q, k, v, scale=scale, causal=isinstance(mask, str) and q.shape[2] > 1)
    prev = _PREV or _ORIG_SDPA
    return prev(q, k, v, scale=scale, mask=mask, sinks=sinks, **kw)


@contextlib.contextmanager
def multirow_attention(cfg: MultirowConfig | None):
    """Route eligible ``fast.scaled_dot_product_attention`` calls through the kernel while
    active; everything else falls through to what was installed before. No-op when ``cfg``
    is None or the patch is already installed."""
    global _ACTIVE, _PREV
    if cfg is None or fast.scaled_dot_product_attention is _patched_call:
        yield
        return
    prev = fast.scaled_dot_product_attention
    prev_cfg, prev_prev = _ACTIVE, _PREV
    _ACTIVE, _PREV = cfg, prev
    fast.scaled_dot_product_attention = _patched_call
    try:
        yield
    finally:
        fast.scaled_dot_product_attention = prev
        _ACTIVE, _PREV = prev_cfg, prev_prev


def active() -> bool:
    return fast.scaled_dot_product_attention is _patched_call


# ---- measurement (multirow_attn.py:391-488) ------------------------------------------

PROBE_Q = (2, 4, 6, 8, 12, 16)
PROBE_KV = (1024, 4096, 16384)
WIN = 1.05


def _chain_ms(fn, q0, kvs, iters: int = 4) -> float:
    """ms per call over a DEPENDENT chain (each output is the next query) across rotated KV sets."""
    import time

    def run():
        q = q0
        for _ in range(iters):
            for kk, vv in kvs:
                q = fn(q, kk, vv)
        return q

    run()
    torch.cuda.synchronize()
    t = time.perf_counter()
    run()
    torch.cuda.synchronize()
    return (time.perf_counter() - t) * 1e3 / (iters * len(kvs))


def measure_window(hq: int, hk: int, d: int, *, dtype=torch.bfloat16, device="cuda", verbose: bool = False,
                   probe_q=PROBE_Q, probe_kv=PROBE_KV) -> tuple[dict | None, dict]:
    """Race the kernel against the stock path on this GPU for shape (hq, hk, d) and return
    ``(window, report)``. Numerics at every probe against an fp32 reference: the kernel's max
    |d| must stay within 2x the stock path's + 2e-3, or the shape is refused. ``max_q`` is the
    widest probed q such that every probed q <= it wins by > 5% at the deepest KV; ``min_kv``
    the shortest probed KV from which that range wins at every deeper probe."""
    if d not in HEAD_DIMS or hk == 0 or hq % hk or dtype not in _DTYPES:
        return None, {"reason": "shape"}
    scale = 1.0 / math.sqrt(d)
    report: dict = {"shape": f"{hq}x{hk}x{d}", "points": {}}
    wins_at: dict[int, list[int]] = {}
    g = torch.Generator(device=device)
    g.manual_seed(0)
    try:
        for kv in probe_kv:
            kvs = [(torch.randn((1, hk, kv, d), generator=g, device=device).to(dtype),
                    torch.randn((1, hk, kv, d), generator=g, device=device).to(dtype)) for _ in range(3)]
            ok = []
            for ql in probe_q:
                if (hq // hk) * ql > MAX_ROWS:
                    report["points"][f"q{ql}@{kv}"] = "unavailable"
                    break
                q = torch.randn((1, hq, ql, d), generator=g, device=device).to(dtype)
                k0, v0 = kvs[0]
                ref = _ORIG_SDPA(q.float(), k0.float(), v0.float(), scale=scale, mask="causal")
                o_m = multirow_sdpa(q, k0, v0, scale=scale, causal=True)
                e_m = float((o_m.float() - ref).abs().max())
                o_x = _ORIG_SDPA(q, k0, v0, scale=scale, mask="causal")
                e_x = float((o_x.float() - ref).abs().max())
                if math.isnan(e_m) or e_m > 2.0 * e_x + 2e-3:
                    report["reason"] = f"numerics q{ql} kv{kv}: {e_m:.4g} vs stock {e_x:.4g}"
                    return None, report
                t_x = _chain_ms(lambda qq, kk, vv: _ORIG_SDPA(qq, kk, vv, scale=scale, mask="causal"), q, kvs)
                t_m = _chain_ms(lambda qq, kk, vv: multirow_sdpa(qq, kk, vv, scale=scale, causal=True), q, kvs)
                report["points"][f"q{ql}@{kv}"] = round(t_x / t_m, 2)
                if t_x > WIN * t_m:
                    ok.append(ql)
            wins_at[kv] = ok
            del kvs
    except Exception as e:  # noqa: BLE001 - a kernel that will not run here is simply off
        report["reason"] = f"kernel unavailable: {type(e).__name__}: {e}"
        return None, report
    deep = wins_at[probe_kv[-1]]
    max_q = 0
    for ql in probe_q:
        if ql not in deep:
            break
        max_q = ql
    if not max_q:
        report["reason"] = "no win on this GPU"
        return None, report
    qs = [ql for ql in probe_q if ql <= max_q]
    min_kv = probe_kv[-1]
    for kv in reversed(probe_kv):
        if all(ql in wins_at[kv] for ql in qs):
            min_kv = kv
        else:
            break
    return {"min_q": probe_q[0], "max_q": max_q, "min_kv": min_kv}, report
