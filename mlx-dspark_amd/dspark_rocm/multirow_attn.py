"""Multi-row verify attention: the gfx950 kernel behind the reference's ``multirow_sdpa`` and
its scoped patch of the attention entry points (plain and quantized-cache).

Same API as the reference module (multirow_attn.py:204-488): ``plan``, ``multirow_sdpa``,
``Window``, ``MultirowConfig``, ``eligible``, ``tree_mask``, ``multirow_attention``,
``active`` and ``measure_window``. The kernel is ``dspark_verify_attention_typed`` (split-KV
pass plus combine, v_mfma_f32_16x16x32_{bf16,f16}); it serves bf16 and fp16, any head_dim
d % 8 == 0 up to 256 (the reference's rule, multirow_attn.py:200-214, :294-307; instances at 64,
128 and 256, smaller head dims zero-padded on chip), whole GQA groups with
gqa * q_len <= 256, and reads K/V through their batch/head/sequence strides (KV-cache views
sliced along the sequence axis are used in place). ``quantized_sdpa`` runs the same kernel
over mlx-lm's quantized-cache triples (``dspark_verify_attention_quantized``).

``multirow_attention(cfg)`` patches :func:`dspark_rocm.fast.scaled_dot_product_attention`:
an eligible call of a measured shape (its :class:`Window`) runs the kernel — causal iff the
mask is the string "causal" and q_len > 1 — and every other call falls through to whatever
was installed before (the split scope, then the stock path) (multirow_attn.py:338-370). A
tree verify registers its exact mask object with :func:`tree_mask`; calls carrying that
object take the kernel's ancestry variant (multirow_attn.py:322-349). The scope also patches
:func:`dspark_rocm.fast.quantized_scaled_dot_product_attention`, mlx-lm's helper for caches
with ``bits``, so a quantized cache of a measured shape runs the kernel too.
"""

from __future__ import annotations

import contextlib
import ctypes
import math
from dataclasses import dataclass

import torch

from . import _lib, _scope, fast, gate, ops

_STOCK = fast.STOCK

MAX_D = 256
MAX_ROWS = 256          # gqa * q_len the kernel's row tiles cover
_DTYPES = tuple(ops.ATTN_DTYPES)


def plan(hq: int, hk: int, q_len: int, d: int, kv_len: int, batch: int = 1) -> dict:
    """Launch geometry of the kernel for this shape (host query): rows R, padded rows RP, row
    groups NRG, keys per block CHUNK, key blocks NB and pass-1 workgroups."""
    out = (ctypes.c_int32 * 6)()
    _lib.check("dspark_verify_attention_plan",
               _lib.load().dspark_verify_attention_plan(batch, hq, hk, q_len, d, kv_len, out))
    return {"R": out[0], "RP": out[1], "NRG": out[2], "CHUNK": out[3], "NB": out[4], "workgroups": out[5]}


def quantized_sdpa(q: torch.Tensor, q_keys, q_values, *, scale: float, causal: bool, group_size: int = 64,
                   bits: int = 8) -> torch.Tensor:
    """The kernel over quantized K/V triples (words, scales, biases) of mlx-lm's
    ``QuantizedKVCache`` (``ops.verify_attention_quantized``)."""
    return ops.verify_attention_quantized(q, q_keys, q_values, scale=scale, causal=causal, bits=bits,
                                          group_size=group_size)


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
        return next((w for w in self.windows if (w.hq, w.hk, w.d) == (hq, hk, d)), None)


def why_not(q, k, v, mask, sinks, cfg: MultirowConfig) -> str | None:
    """The first reason the kernel cannot serve this call, or None when it can (device aside).

    The conditions are the reference's gate (multirow_attn.py:288-312) plus what torch lets
    us check that mlx does not expose: K/V must be contiguous along head_dim (any batch, head
    and sequence strides are fine, e.g. a cache view sliced along the sequence)."""
    if sinks is not None:
        return "sinks"
    if mask is not None and not (isinstance(mask, str) and mask == "causal"):
        return "mask"
    if not (q.dim() == k.dim() == v.dim() == 4):
        return "rank"
    B, Hq, q_len, D = q.shape
    Hk, L = k.shape[1], k.shape[2]
    w = cfg.window(Hq, Hk, D)
    if w is None:
        return "unmeasured shape"
    if not w.min_q <= q_len <= min(w.max_q, L):
        return "q_len outside the window"
    if L < max(w.min_kv, 16):
        return "kv_len below the window"
    if not (q.dtype in _DTYPES and k.dtype == v.dtype == q.dtype):
        return "dtype"
    if not ops.attn_head_dim_ok(D) or k.shape[-1] != D or v.shape[-1] != D:
        return "head_dim"
    if Hk == 0 or Hq % Hk or tuple(v.shape[:3]) != (B, Hk, L) or k.shape[0] != B:
        return "heads"
    if (Hq // Hk) * q_len > MAX_ROWS:
        return "rows"
    if k.stride(-1) != 1 or v.stride(-1) != 1:
        return "head_dim stride"
    return None


def eligible_shape(q, k, v, mask, sinks, cfg: MultirowConfig) -> bool:
    """Everything :func:`eligible` checks except the device."""
    return why_not(q, k, v, mask, sinks, cfg) is None


def eligible(q, k, v, mask, sinks, cfg: MultirowConfig) -> bool:
    """Structural + window check on GPU tensors (multirow_attn.py:288-312)."""
    return q.is_cuda and k.is_cuda and v.is_cuda and eligible_shape(q, k, v, mask, sinks, cfg)


# Scope state: the active config, what the patch falls through to, the registered tree mask.
_config = _scope.Slot()
_fallthrough = _scope.Slot()
_fallthrough_q = _scope.Slot()
_tree = _scope.Slot()


def current_tree():
    """``(mask, anc_bits)`` registered by the innermost :func:`tree_mask`, or None."""
    return _tree.value


@contextlib.contextmanager
def tree_mask(mask, anc_bits: torch.Tensor):
    """Declare ``mask`` (the exact object a tree verify passes) as a tree-verify mask whose
    visibility over the last W keys is ``anc_bits`` (uint32 per row). Calls carrying that
    object take the kernel's ancestry variant; the match is by identity (multirow_attn.py:319-335)."""
    with _tree.holding((mask, anc_bits)):
        yield


def _route(q, k, v, scale, mask, sinks, cfg):
    """The kernel's answer for this call, or None when it does not serve it."""
    tree = _tree.value
    if tree is not None and mask is tree[0]:
        if q.dim() == 4 and q.shape[2] <= 32 and eligible(q, k, v, None, sinks, cfg):
            return multirow_sdpa(q, k, v, scale=scale, causal=False, tree_anc=tree[1])
        return None
    if eligible(q, k, v, mask, sinks, cfg):
        return multirow_sdpa(q, k, v, scale=scale, causal=mask == "causal" and q.shape[2] > 1)
    return None


def why_not_quantized(q, q_keys, q_values, mask, cfg: MultirowConfig, group_size: int, bits: int) -> str | None:
    """:func:`why_not` for a quantized-cache call: the same window and shape rules, on the
    (words, scales, biases) triples, plus the triples' own layout (every shape, unit last
    strides, scales and biases sharing strides), so a malformed triple falls through to the
    stock path instead of raising inside the scope."""
    if bits not in ops.KV_BITS or group_size != 64:
        return "format"
    kw, ks, kb = q_keys
    vw, vs, vb = q_values
    if not all(t.dim() == 4 for t in (kw, ks, kb, vw, vs, vb)) or q.dim() != 4:
        return "rank"
    D = q.shape[-1]
    if D not in ops.QUANT_HEAD_DIMS:
        return "head_dim"
    k_like = torch.empty((kw.shape[0], kw.shape[1], kw.shape[2], D), dtype=ks.dtype, device="meta")
    reason = why_not(q, k_like, k_like, mask, None, cfg)
    if reason:
        return reason
    lead = tuple(kw.shape[:3])
    if kw.shape[-1] * 32 // bits != D or tuple(vw.shape) != tuple(kw.shape):
        return "head_dim"
    G = D // group_size
    if any(tuple(t.shape) != lead + (G,) for t in (ks, kb, vs, vb)):
        return "scales"
    if any(t.stride(-1) != 1 for t in (kw, ks, kb, vw, vs, vb)):
        return "last-dim stride"
    if ks.stride() != kb.stride() or vs.stride() != vb.stride():
        return "scale/bias strides"
    if any(t.dtype not in (torch.int32, torch.uint32) for t in (kw, vw)):
        return "word dtype"
    if not (ks.dtype == kb.dtype == vs.dtype == vb.dtype == q.dtype):
        return "dtype"
    return None


def _patched_quantized(q, q_keys, q_values, *, scale, mask=None, group_size: int = 64, bits: int = 8):
    cfg = _config.value
    if (cfg is not None and q.is_cuda and q_keys[0].is_cuda
            and why_not_quantized(q, q_keys, q_values, mask, cfg, group_size, bits) is None):
        return quantized_sdpa(q, q_keys, q_values, scale=scale, causal=mask == "causal" and q.shape[2] > 1,
                              group_size=group_size, bits=bits)
    below = _fallthrough_q.value or fast.QUANTIZED_STOCK
    return below(q, q_keys, q_values, scale=scale, mask=mask, group_size=group_size, bits=bits)


def _patched_call(q, k, v, *, scale, mask=None, sinks=None, **kw):
    cfg = _config.value
    out = _route(q, k, v, scale, mask, sinks, cfg) if cfg is not None and not kw else None
    if out is not None:
        return out
    below = _fallthrough.value or _STOCK
    return below(q, k, v, scale=scale, mask=mask, sinks=sinks, **kw)


@contextlib.contextmanager
def multirow_attention(cfg: MultirowConfig | None):
    """Route eligible ``fast.scaled_dot_product_attention`` calls through the kernel while
    active; every other call goes to whatever was installed before (the split scope, then the
    stock path). No-op when ``cfg`` is None or the patch is already installed."""
    if cfg is None or active():
        yield
        return
    below, below_q = fast.scaled_dot_product_attention, fast.quantized_scaled_dot_product_attention
    with _config.holding(cfg), _fallthrough.holding(below), _fallthrough_q.holding(below_q), \
            _scope.replaced(fast, "scaled_dot_product_attention", _patched_call), \
            _scope.replaced(fast, "quantized_scaled_dot_product_attention", _patched_quantized):
        yield


def active() -> bool:
    return fast.scaled_dot_product_attention is _patched_call


# ---- measurement (the reference's gate: multirow_attn.py:391-488) --------------------

PROBE_Q = (2, 4, 6, 8, 12, 16)
PROBE_KV = (1024, 4096, 16384)
WIN = 1.05


def _window_from_wins(wins: dict[int, set[int]], probe_q, probe_kv) -> dict | None:
    """The served window from the set of winning q at each probed kv length: ``max_q`` ends
    the longest run of winning probe q (from the smallest) at the deepest kv; ``min_kv`` is
    the shortest kv from which every deeper probe also wins that whole run."""
    deepest = wins.get(probe_kv[-1], set())
    run = []
    for ql in probe_q:
        if ql not in deepest:
            break
        run.append(ql)
    if not run:
        return None
    min_kv = probe_kv[-1]
    for kv in sorted(probe_kv, reverse=True):
        if not set(run) <= wins.get(kv, set()):
            break
        min_kv = kv
    return {"min_q": probe_q[0], "max_q": run[-1], "min_kv": min_kv}


def measure_window(hq: int, hk: int, d: int, *, dtype=torch.bfloat16, device="cuda", verbose: bool = False,
                   probe_q=PROBE_Q, probe_kv=PROBE_KV) -> tuple[dict | None, dict]:
    """Race the kernel against the stock path for shape (hq, hk, d) on this GPU; returns
    ``(window, report)``. At every probe (q_len, kv_len) the kernel's max |d| from an fp32
    reference must stay within twice the stock path's plus 2e-3, or the shape is refused; the
    kernel wins a probe when the stock path takes more than ``WIN`` times as long (HIP-event
    chains over three KV sets). ``window`` is None when nothing wins or the kernel cannot run."""
    if not ops.attn_head_dim_ok(d) or hk == 0 or hq % hk or dtype not in _DTYPES:
        return None, {"reason": "shape"}
    scale = d ** -0.5
    report: dict = {"shape": f"{hq}x{hk}x{d}", "points": {}}
    wins: dict[int, set[int]] = {}
    gen = torch.Generator(device=device)
    gen.manual_seed(0)

    def rand(*shape):
        return torch.randn(shape, generator=gen, device=device).to(dtype)

    try:
        for kv in probe_kv:
            sets = [(rand(1, hk, kv, d), rand(1, hk, kv, d)) for _ in range(3)]
            wins[kv] = set()
            for ql in probe_q:
                if (hq // hk) * ql > MAX_ROWS:
                    report["points"][f"q{ql}@{kv}"] = "unavailable"
                    break
                q = rand(1, hq, ql, d)
                kk, vv = sets[0]
                exact = _STOCK(q.float(), kk.float(), vv.float(), scale=scale, mask="causal")
                e_kernel = gate.max_abs_diff(multirow_sdpa(q, kk, vv, scale=scale, causal=True), exact)
                e_stock = gate.max_abs_diff(_STOCK(q, kk, vv, scale=scale, mask="causal"), exact)
                if not e_kernel <= 2.0 * e_stock + 2e-3:
                    report["reason"] = f"numerics q{ql} kv{kv}: {e_kernel:.4g} vs stock {e_stock:.4g}"
                    return None, report
                ratio = gate.speedup(
                    [lambda a=a, b=b: _STOCK(q, a, b, scale=scale, mask="causal") for a, b in sets],
                    [lambda a=a, b=b: multirow_sdpa(q, a, b, scale=scale, causal=True) for a, b in sets])
                report["points"][f"q{ql}@{kv}"] = round(ratio, 2)
                if ratio > WIN:
                    wins[kv].add(ql)
            del sets
    except Exception as e:  # noqa: BLE001 - a kernel that will not run here is simply off
        report["reason"] = f"kernel unavailable: {type(e).__name__}: {e}"
        return None, report
    window = _window_from_wins(wins, tuple(probe_q), tuple(probe_kv))
    if window is None:
        report["reason"] = "no win on this GPU"
    if verbose:
        print(f"  multirow attention {report['shape']}: {window} {report['points']}", flush=True)
    return window, report
