"""Load-time wiring of the verify kernels: each kernel's gate is measured once per machine, the
verdict is cached on disk, and the process-wide settings that the dispatch scopes read are set
from it for a loaded target (and drafter).

Entry points (names, signatures and meaning as the reference's calibrate.py:933-985,
:1062-1153, :1222-1302, :1352-1407):

* ``small_m_qmm_shapes`` / ``apply_small_m`` -- the weight-shape keys whose small-M kernel
  passes :func:`dspark_rocm.small_m_qmm.measure_shapes`, turned into the instance allowlist
  :data:`SMALL_M_IDS`;
* ``multirow_windows`` / ``apply_multirow_attn`` -- one measured
  :class:`~dspark_rocm.multirow_attn.Window` per attention shape (the target's and a DSpark
  drafter's context attention), stored as :data:`MULTIROW_CFG`;
* ``measure_split_window`` / ``apply_sdpa_split`` -- the row-split window of the stock
  attention path (:data:`SDPA_SPLIT_CFG`), on only where splitting a wide verify call is
  measured to be faster;
* ``wide_gemm_min_rows`` / ``apply_wide_gemm`` -- the prefill wide path's crossover and
  verified shapes (:data:`WIDE_GEMM_MIN_ROWS` / :data:`WIDE_GEMM_SHAPES`);
* :func:`verify_scopes` -- the scopes a verify loop runs under, in the reference's order
  (generate.py:52-83): row split outermost, multi-row attention inside it (calls it does not
  serve fall through to the split), then the small-M allowlist.

Every measurement goes through one helper, :func:`verdict`: a :class:`Probe` names what is
measured (its kind and subject), how, how to report it, and when a cached value no longer
describes the live models. Verdicts are JSON files keyed by the GPU (name, gfx target) and this
library's version. Nothing here raises on a kernel failure: a shape that cannot run stays on
the stock path. (The reference also gates kernels by Apple GPU generation, calibrate.py:1053-1059
and :1311-1314; MI355X has no such gate.)
"""

from __future__ import annotations

import contextlib
import hashlib
import json
import os
from dataclasses import dataclass
from typing import Any, Callable

SCHEMA = 1

SMALL_M_IDS: frozenset | None = None     # allowlist routed through the small-M qmm kernel
WIDE_GEMM_MIN_ROWS: int | None = None    # prefill wide path threshold (None: off)
WIDE_GEMM_SHAPES: list | None = None     # its verified shape keys
MULTIROW_CFG = None                      # multirow_attn.MultirowConfig, or None
SDPA_SPLIT_CFG = None                    # sdpa_split.SplitConfig, or None


# ------------------------------------------------------------------ verdict cache

def cache_dir(path: str | None = None) -> str:
    """Where verdicts live: ``path``, else $DSPARK_CACHE_DIR, else ~/.cache/dspark_rocm."""
    return path or os.environ.get("DSPARK_CACHE_DIR") or os.path.join(os.path.expanduser("~"), ".cache",
                                                                      "dspark_rocm")


def _file(key: str, path: str | None) -> str:
    return os.path.join(cache_dir(path), hashlib.sha1(key.encode()).hexdigest()[:20] + ".json")


def load_cached(key: str, path: str | None = None):
    try:
        with open(_file(key, path)) as f:
            entry = json.load(f)
    except (OSError, ValueError):
        return None
    return entry.get("value") if entry.get("key") == key else None


def save_cached(key: str, value, path: str | None = None) -> None:
    try:
        os.makedirs(cache_dir(path), exist_ok=True)
        tmp = _file(key, path) + ".tmp"
        with open(tmp, "w") as f:
            json.dump({"key": key, "value": value}, f)
        os.replace(tmp, _file(key, path))
    except OSError:
        pass            # an unwritable cache only costs a re-measurement next time


def device_key() -> str:
    """The GPU and library a verdict holds for."""
    import torch

    from . import _lib

    dev = "cpu"
    if torch.cuda.is_available():
        p = torch.cuda.get_device_properties(0)
        dev = f"{p.name}|{getattr(p, 'gcnArchName', '')}"
    try:
        lib = (_lib.load().dspark_version() or b"").decode()
    except _lib.DsparkUnavailable:
        lib = "unbuilt"
    return f"v{SCHEMA}|{dev}|{lib}"


@dataclass(frozen=True)
class Probe:
    """One cached measurement: ``kind`` and ``subject`` make its cache key; ``measure()``
    returns a JSON-serialisable value; ``report(value)`` says what it means for the log;
    ``stale(value)`` tells a cached value that no longer fits the live models (measured again)."""
    kind: str
    subject: str
    measure: Callable[[], Any]
    report: Callable[[Any], str]
    stale: Callable[[Any], bool] = lambda value: False


def verdict(probe: Probe, *, cache_dir: str | None = None, refresh: bool = False, verbose: bool = True):
    """The probe's value: cached for this GPU and library when present and not stale, else
    measured now and cached (``refresh`` always measures)."""
    key = f"{device_key()}|{probe.kind}|{probe.subject}"
    value = None if refresh else load_cached(key, cache_dir)
    if value is not None and not probe.stale(value):
        return value
    if verbose:
        print(f"measuring {probe.kind} for {probe.subject} (once on this machine, then cached)", flush=True)
    value = probe.measure()
    save_cached(key, value, cache_dir)
    if verbose:
        print(f"  {probe.kind}: {probe.report(value)}", flush=True)
    return value


def _model_of(obj):
    """The network inside a Target-like wrapper (``.model``), or the object itself."""
    return getattr(obj, "model", obj)


# ------------------------------------------------------------------ small-M qmm

def _small_m_probe(target, drafter, target_repo, drafter_repo) -> Probe:
    from . import small_m_qmm

    model = _model_of(target)
    return Probe(
        "smallm", f"{target_repo}|{drafter_repo}",
        measure=lambda: list(small_m_qmm.measure_shapes(model, drafter, verbose=False)),
        report=lambda keys: f"{len(keys)} weight shapes take the kernel" if keys else "every shape stays stock",
        # keys written under another key format match no live module (calibrate.py:1136-1150)
        stale=lambda keys: bool(keys) and not small_m_qmm.ids_for_shapes(keys, model, drafter))


def small_m_qmm_shapes(target, drafter=None, *, target_repo: str, drafter_repo: str | None = None,
                       cache_dir: str | None = None, refresh: bool = False, verbose: bool = True) -> list[str]:
    """Weight-shape keys whose verify-window forwards should run on the small-M kernel here,
    measured once and cached (``refresh`` measures again and overwrites)."""
    probe = _small_m_probe(target, drafter, target_repo, drafter_repo)
    return list(verdict(probe, cache_dir=cache_dir, refresh=refresh, verbose=verbose))


def apply_small_m(target, drafter=None, *, target_repo: str, drafter_repo: str | None = None,
                  enabled: bool | None = None, cache_dir: str | None = None, verbose: bool = True):
    """Turn the small-M kernel on for this process (:data:`SMALL_M_IDS`) and return the
    allowlist, or None when off. ``enabled=None`` measures (cached); False disables."""
    global SMALL_M_IDS
    from .small_m_qmm import ids_for_shapes

    SMALL_M_IDS = None
    if enabled is not False:
        keys = small_m_qmm_shapes(target, drafter, target_repo=target_repo, drafter_repo=drafter_repo,
                                  cache_dir=cache_dir, verbose=verbose)
        SMALL_M_IDS = ids_for_shapes(keys, _model_of(target), drafter) or None
    return SMALL_M_IDS


# ------------------------------------------------------------------ attention shapes

def _attn_dims(target):
    """(query heads, KV heads, head dim) of the target's attention layers, or None."""
    args = getattr(_model_of(target), "args", None)
    if args is None:
        return None
    field = args.get if isinstance(args, dict) else (lambda name: getattr(args, name, None))
    hq = field("num_attention_heads")
    hk = field("num_key_value_heads") or hq
    width = field("hidden_size")
    d = field("head_dim") or (width // hq if hq and width else None)
    return (int(hq), int(hk), int(d)) if hq and hk and d else None


# what keeps a DSpark drafter's context attention off the kernel: a causal block, a sliding
# window or attention sinks (its calls then carry array masks), or no context update at all
# (calibrate.py:1315-1327)
_DRAFTER_BLOCKERS = ("causal_block", "sliding_window", "sink")
_DRAFTER_NEEDS = ("n_heads", "n_kv_heads", "head_dim", "update_ctx")


def _drafter_attn_dims(drafter):
    """(query heads, KV heads, head dim) of a DSpark drafter's context attention when it can
    take the kernel, else None."""
    layers = list(getattr(drafter, "layers", None) or [])
    attn = getattr(layers[0], "self_attn", None) if layers else None
    if attn is None or not all(hasattr(attn, n) for n in _DRAFTER_NEEDS):
        return None
    if any(getattr(attn, n, None) for n in _DRAFTER_BLOCKERS):
        return None
    return int(attn.n_heads), int(attn.n_kv_heads), int(attn.head_dim)


def _attention_shapes(target, drafter) -> list[tuple[int, int, int]]:
    """The distinct attention shapes of the target and a DSpark drafter, target first."""
    found = (_attn_dims(target), _drafter_attn_dims(drafter) if drafter is not None else None)
    return list(dict.fromkeys(s for s in found if s))


# ------------------------------------------------------------------ multi-row attention

def multirow_windows(shapes, *, cache_dir: str | None = None, refresh: bool = False, verbose: bool = True) -> list:
    """One measured :class:`~dspark_rocm.multirow_attn.Window` per (hq, hk, d) that wins here
    (each raced and checked once, cached)."""
    from . import multirow_attn

    def probe(hq, hk, d):
        def measure():
            window, report = multirow_attn.measure_window(hq, hk, d, verbose=False)
            return {"window": window, "report": report}

        return Probe("multirow", f"{hq}x{hk}x{d}", measure,
                     report=lambda v: (f"q {v['window']['min_q']}..{v['window']['max_q']} from "
                                       f"{v['window']['min_kv']} keys" if v.get("window") else
                                       f"stock ({(v.get('report') or {}).get('reason', 'no win')})"))

    measured = [(s, verdict(probe(*s), cache_dir=cache_dir, refresh=refresh, verbose=verbose)) for s in shapes]
    return [multirow_attn.Window(*s, **v["window"]) for s, v in measured if v.get("window")]


def apply_multirow_attn(target, drafter=None, *, enabled: bool | None = None, cache_dir: str | None = None,
                        verbose: bool = True):
    """Turn the multi-row attention kernel on for this process (:data:`MULTIROW_CFG`) for the
    target's and a DSpark drafter's attention shapes; returns the config, or None when off."""
    global MULTIROW_CFG
    from .multirow_attn import MultirowConfig

    MULTIROW_CFG = None
    if enabled is not False:
        windows = multirow_windows(_attention_shapes(target, drafter), cache_dir=cache_dir, verbose=verbose)
        MULTIROW_CFG = MultirowConfig(tuple(windows)) if windows else None
    return MULTIROW_CFG


# ------------------------------------------------------------------ row split of the stock path

SPLIT_PROBE_KEYS = 16384      # keys of the probe's synthetic cache
SPLIT_MARGIN = 0.05           # a split width must save at least this fraction of the call


def split_window_from_costs(cost: dict, max_chunk: int, *, min_kv: int = 4096,
                            margin: float = SPLIT_MARGIN) -> dict | None:
    """The split window a cost sweep implies (``cost[q]`` = one stock call of q rows), or None.

    Width q gains when the blocks :func:`sdpa_split._partition` cuts it into cost, together,
    less than ``(1 - margin) * cost[q]``. The window is the first run of consecutive gaining
    widths above ``max_chunk`` (a lone gain after a gap is timing noise)."""
    from .sdpa_split import _partition

    def gains(q):
        return q in cost and sum(cost[s] for s in _partition(q, max_chunk)) < (1.0 - margin) * cost[q]

    q = max_chunk + 1
    top = max(cost) if cost else 0
    while q <= top and not gains(q):
        q += 1
    if q > top:
        return None
    first = q
    while q + 1 <= top and gains(q + 1):
        q += 1
    return {"min_q": first, "max_q": q, "min_kv": min_kv, "max_chunk": max_chunk}


def _stock_attention_costs(hq: int, hk: int, d: int, widths=range(1, 17), keys: int = SPLIT_PROBE_KEYS) -> dict:
    """Milliseconds of one stock attention call per q_len (causal, bf16, over ``keys`` keys;
    HIP events over back-to-back calls rotating two KV sets)."""
    import torch

    from . import fast, gate

    dev = torch.device("cuda")
    g = torch.Generator(device=dev)
    g.manual_seed(hq * 131 + d)
    kv = [(torch.randn((1, hk, keys, d), generator=g, device=dev).to(torch.bfloat16),
           torch.randn((1, hk, keys, d), generator=g, device=dev).to(torch.bfloat16)) for _ in range(2)]
    out = {}
    for q_len in widths:
        q = torch.randn((1, hq, q_len, d), generator=g, device=dev).to(torch.bfloat16)
        calls = [lambda k=k, v=v: fast.STOCK(q, k, v, scale=d ** -0.5, mask="causal") for k, v in kv]
        out[q_len] = min(gate.chain_ms(calls) for _ in range(3))
    return out


def _split_chunk(cost: dict, limit: int = 8) -> int:
    """The block size of the split: the width up to ``limit`` with the lowest cost per row (the
    stock path's most efficient width on this machine)."""
    candidates = [q for q in cost if q <= limit]
    return min(candidates, key=lambda q: (cost[q] / q, -q)) if candidates else 1


def measure_split_window(hq: int, hk: int, d: int, *, cache_dir: str | None = None, refresh: bool = False,
                         verbose: bool = True) -> dict | None:
    """The row-split window ``{min_q, max_q, min_kv, max_chunk}`` of the stock attention path
    for this shape on this machine, or None where splitting never pays (cached)."""
    def measure():
        try:
            cost = _stock_attention_costs(hq, hk, d)
        except Exception as e:  # noqa: BLE001 - no device or no memory: the split stays off
            return {"window": None, "reason": f"{type(e).__name__}: {e}"}
        return {"window": split_window_from_costs(cost, _split_chunk(cost)), "cost_ms": cost}

    probe = Probe("split", f"{hq}x{hk}x{d}", measure,
                  report=lambda v: (f"rows {v['window']['min_q']}..{v['window']['max_q']} in blocks of "
                                    f"{v['window']['max_chunk']}" if v.get("window") else "no gain: off"))
    return verdict(probe, cache_dir=cache_dir, refresh=refresh, verbose=verbose).get("window")


def apply_sdpa_split(target, *, target_repo: str | None = None, enabled: bool | None = None,
                     cache_dir: str | None = None, verbose: bool = True):
    """Turn the row split of the stock attention path on for this process
    (:data:`SDPA_SPLIT_CFG`) and return its :class:`~dspark_rocm.sdpa_split.SplitConfig`, or
    None when off. ``enabled=None`` measures (cached); False disables; True takes the default
    window without measuring, as does a target whose attention shape cannot be read."""
    global SDPA_SPLIT_CFG
    from .sdpa_split import SplitConfig

    dims = _attn_dims(target) if enabled is None else None
    if enabled is False:
        SDPA_SPLIT_CFG = None
    elif enabled is True or dims is None:
        SDPA_SPLIT_CFG = SplitConfig()
    else:
        window = measure_split_window(*dims, cache_dir=cache_dir, verbose=verbose)
        SDPA_SPLIT_CFG = SplitConfig(**window) if window else None
    return SDPA_SPLIT_CFG


# ------------------------------------------------------------------ prefill wide path

def wide_gemm_min_rows(target, drafter=None, *, target_repo: str, cache_dir: str | None = None,
                       refresh: bool = False, verbose: bool = True) -> tuple[int | None, list[str]]:
    """``(min_rows, shape keys)`` from which prefill forwards take the wide path here, or
    ``(None, [])`` when it never pays or no shape verifies; measured once (the drafter's
    projections run at prefill width too, so its shapes are verified with the target's) and
    cached."""
    from . import wide_gemm

    def measure():
        try:
            found = wide_gemm.measure_crossover(_model_of(target), drafter)
        except Exception as e:  # noqa: BLE001 - a kernel that will not launch leaves prefill on stock
            return {"min_rows": None, "shapes": [], "reason": f"{type(e).__name__}: {e}"}
        min_rows, shapes = found if found else (None, [])
        return {"min_rows": min_rows, "shapes": list(shapes)}

    probe = Probe("widegemm", target_repo, measure,
                  report=lambda v: (f"prefill projections of >= {v['min_rows']} rows, {len(v['shapes'])} shapes, "
                                    "bit-identical to stock" if v.get("min_rows") else
                                    f"stock ({v.get('reason', 'never faster, or no shape exact')})"))
    entry = verdict(probe, cache_dir=cache_dir, refresh=refresh, verbose=verbose)
    return entry.get("min_rows"), list(entry.get("shapes") or [])


def apply_wide_gemm(target, drafter=None, *, target_repo: str, min_rows: int | None = None,
                    cache_dir: str | None = None, verbose: bool = True) -> int | None:
    """Turn the prefill wide path on for this process (:data:`WIDE_GEMM_MIN_ROWS`,
    :data:`WIDE_GEMM_SHAPES`) and return the threshold. ``min_rows=None`` measures (cached),
    0 disables, N forces N -- raised to the path's floor and still only for the shapes that
    verify there."""
    global WIDE_GEMM_MIN_ROWS, WIDE_GEMM_SHAPES
    from . import wide_gemm

    if min_rows is None:
        WIDE_GEMM_MIN_ROWS, WIDE_GEMM_SHAPES = wide_gemm_min_rows(target, drafter, target_repo=target_repo,
                                                                  cache_dir=cache_dir, verbose=verbose)
        return WIDE_GEMM_MIN_ROWS
    forced = max(int(min_rows), wide_gemm.SAFE_MIN_ROWS) if int(min_rows) else None
    WIDE_GEMM_MIN_ROWS = forced
    WIDE_GEMM_SHAPES = wide_gemm.verified_shapes([_model_of(target), drafter], forced) if forced else []
    return WIDE_GEMM_MIN_ROWS


# ------------------------------------------------------------------ scopes

@contextlib.contextmanager
def verify_scopes():
    """The dispatch scopes of a verify loop from the process-wide settings above (each a no-op
    when its setting is None): row split, then multi-row attention, then the small-M qmm."""
    from .multirow_attn import multirow_attention
    from .sdpa_split import sdpa_split
    from .small_m_qmm import small_m_matmul

    with sdpa_split(SDPA_SPLIT_CFG), multirow_attention(MULTIROW_CFG), small_m_matmul(SMALL_M_IDS):
        yield
