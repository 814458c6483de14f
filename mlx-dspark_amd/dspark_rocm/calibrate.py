"""Load-time wiring of the verify kernels: measure each shape's gate once per machine, cache the
verdict, and turn the kernels on for a loaded target (and drafter).

The reference's entry points (calibrate.py:1062-1153 for the small-M qmm, :1352-1407 for the
multi-row attention):

* ``small_m_qmm_shapes(target, drafter, target_repo=...)`` -> the weight-shape keys whose
  kernel passes :func:`dspark_rocm.small_m_qmm.measure_shapes` here; ``apply_small_m`` turns
  them into the instance allowlist and stores it in :data:`SMALL_M_IDS`.
* ``multirow_windows(shapes)`` -> one measured :class:`~dspark_rocm.multirow_attn.Window`
  per attention shape; ``apply_multirow_attn(target, drafter)`` finds the target's and a DSpark
  drafter's attention shapes, measures them and stores the config in :data:`MULTIROW_CFG`.
* ``wide_gemm_min_rows`` / ``apply_wide_gemm(target, drafter)`` measure the prefill wide
  path's crossover and verified shapes (:mod:`dspark_rocm.wide_gemm`) and store them in
  :data:`WIDE_GEMM_MIN_ROWS` / :data:`WIDE_GEMM_SHAPES`, which ``Target.prefill`` reads
  (calibrate.py:933-985).
* :func:`verify_scopes` enters the scopes a verify loop runs under, in the reference's order
  (generate.py:52-83): the row split outermost, the multi-row attention inside it (so calls it
  does not serve fall through to the split), then the small-M allowlist.

Verdicts are cached as JSON, one file per key, keyed by the GPU (name and gfx target) and this
library's version, so a machine measures once. A cached shape list that matches no live module
(a shape-key format change) is measured again (calibrate.py:1136-1150). Nothing here raises on a
kernel failure: a shape that cannot run stays on the stock path. (The reference also gates both
kernels by Apple GPU generation, calibrate.py:1053-1059 and :1311-1314; MI355X has no such
gate.)
"""

from __future__ import annotations

import contextlib
import hashlib
import json
import os

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


# ------------------------------------------------------------------ small-M qmm

def small_m_qmm_shapes(target, drafter=None, *, target_repo: str, drafter_repo: str | None = None,
                       cache_dir: str | None = None, refresh: bool = False, verbose: bool = True) -> list[str]:
    """Weight-shape keys whose verify-window forwards should run on the small-M kernel here,
    measured once and cached (``refresh`` measures again and overwrites)."""
    from . import small_m_qmm

    key = f"{device_key()}|smallm|{target_repo}|{drafter_repo}"
    shapes = None if refresh else load_cached(key, cache_dir)
    if shapes is None:
        if verbose:
            print("calibrating the small-M qmm kernel (once per machine, cached)", flush=True)
        shapes = small_m_qmm.measure_shapes(getattr(target, "model", target), drafter, verbose=verbose)
        save_cached(key, shapes, cache_dir)
        if verbose:
            print(f"  small-M qmm: {'on for ' + str(len(shapes)) + ' weight shapes' if shapes else 'off'}", flush=True)
    return list(shapes)


def apply_small_m(target, drafter=None, *, target_repo: str, drafter_repo: str | None = None,
                  enabled: bool | None = None, cache_dir: str | None = None, verbose: bool = True):
    """Turn the small-M kernel on for this process (:data:`SMALL_M_IDS`) and return the
    allowlist, or None when off. ``enabled=None`` measures (cached); False disables."""
    global SMALL_M_IDS
    from .small_m_qmm import ids_for_shapes

    if enabled is False:
        SMALL_M_IDS = None
        return None
    model = getattr(target, "model", target)
    kw = dict(target_repo=target_repo, drafter_repo=drafter_repo, cache_dir=cache_dir, verbose=verbose)
    shapes = small_m_qmm_shapes(target, drafter, **kw)
    ids = ids_for_shapes(shapes, model, drafter)
    if shapes and not ids:
        # the cached keys match no live module: written under another shape-key format
        shapes = small_m_qmm_shapes(target, drafter, refresh=True, **kw)
        ids = ids_for_shapes(shapes, model, drafter)
    SMALL_M_IDS = ids or None
    return SMALL_M_IDS


# ------------------------------------------------------------------ multi-row attention

def _attn_dims(target):
    """(query heads, KV heads, head dim) of the target's attention layers, or None."""
    model = getattr(target, "model", target)
    args = getattr(model, "args", None)
    if args is None:
        return None
    if isinstance(args, dict):
        get = args.get
    else:
        def get(k, default=None):
            return getattr(args, k, default)
    hq, hk = get("num_attention_heads"), get("num_key_value_heads") or get("num_attention_heads")
    d = get("head_dim") or (get("hidden_size") // hq if hq and get("hidden_size") else None)
    return (int(hq), int(hk), int(d)) if hq and hk and d else None


def _drafter_attn_dims(drafter):
    """(query heads, KV heads, head dim) of a DSpark drafter's context attention when it can
    take the kernel (an unmasked block without sinks: no causal block, sliding window or sink,
    and a context update), else None (calibrate.py:1315-1327)."""
    layers = getattr(drafter, "layers", None) or []
    attn = getattr(layers[0], "self_attn", None) if len(layers) else None
    if attn is None or not all(hasattr(attn, n) for n in ("n_heads", "n_kv_heads", "head_dim", "update_ctx")):
        return None
    if getattr(attn, "causal_block", False) or getattr(attn, "sliding_window", None) or getattr(attn, "sink", False):
        return None
    return int(attn.n_heads), int(attn.n_kv_heads), int(attn.head_dim)


def multirow_windows(shapes, *, cache_dir: str | None = None, refresh: bool = False, verbose: bool = True) -> list:
    """One measured :class:`~dspark_rocm.multirow_attn.Window` per (hq, hk, d) that wins here
    (each raced and checked once, cached)."""
    from .multirow_attn import Window, measure_window

    out = []
    for hq, hk, d in shapes:
        key = f"{device_key()}|multirow|{hq}x{hk}x{d}"
        hit = None if refresh else load_cached(key, cache_dir)
        if hit is None:
            if verbose:
                print(f"calibrating multi-row attention for {hq}x{hk}x{d} (once per machine, cached)", flush=True)
            win, report = measure_window(hq, hk, d, verbose=verbose)
            hit = {"window": win, "report": report}
            save_cached(key, hit, cache_dir)
        if hit.get("window"):
            out.append(Window(hq, hk, d, **hit["window"]))
    return out


def apply_multirow_attn(target, drafter=None, *, enabled: bool | None = None, cache_dir: str | None = None,
                        verbose: bool = True):
    """Turn the multi-row attention kernel on for this process (:data:`MULTIROW_CFG`) for the
    target's and a DSpark drafter's attention shapes; returns the config, or None when off."""
    global MULTIROW_CFG
    from .multirow_attn import MultirowConfig

    if enabled is False:
        MULTIROW_CFG = None
        return None
    shapes = []
    for dims in (_attn_dims(target), _drafter_attn_dims(drafter) if drafter is not None else None):
        if dims and dims not in shapes:
            shapes.append(dims)
    windows = multirow_windows(shapes, cache_dir=cache_dir, verbose=verbose)
    MULTIROW_CFG = MultirowConfig(tuple(windows)) if windows else None
    return MULTIROW_CFG


# ------------------------------------------------------------------ prefill wide path

def wide_gemm_min_rows(target, drafter=None, *, target_repo: str, cache_dir: str | None = None,
                       refresh: bool = False, verbose: bool = True) -> tuple[int | None, list[str]]:
    """``(min_rows, shape keys)`` from which prefill forwards take the wide path here, or
    ``(None, [])`` when it never pays or no shape verifies; measured once (the drafter's
    projections run at prefill width too, so its shapes are verified with the target's) and
    cached (calibrate.py:933-962)."""
    from .wide_gemm import measure_crossover

    key = f"{device_key()}|widegemm|{target_repo}"
    entry = None if refresh else load_cached(key, cache_dir)
    if entry is None:
        if verbose:
            print("calibrating the prefill wide path (once per machine, cached)", flush=True)
        try:
            got = measure_crossover(getattr(target, "model", target), drafter)
        except Exception as e:  # noqa: BLE001 - a kernel that will not launch leaves prefill on stock
            if verbose:
                print(f"  prefill wide path: off (kernel unavailable: {type(e).__name__}: {e})", flush=True)
            got = None
        entry = {"min_rows": got[0], "shapes": got[1]} if got else {"min_rows": None, "shapes": []}
        save_cached(key, entry, cache_dir)
        if verbose:
            state = (f"on from M={entry['min_rows']} for {len(entry['shapes'])} weight shapes (verified bit-identical)"
                     if entry["min_rows"] else "off (no gain, or not exact here)")
            print(f"  prefill wide path: {state}", flush=True)
    return entry.get("min_rows"), list(entry.get("shapes") or [])


def apply_wide_gemm(target, drafter=None, *, target_repo: str, min_rows: int | None = None,
                    cache_dir: str | None = None, verbose: bool = True) -> int | None:
    """Turn the prefill wide path on for this process (:data:`WIDE_GEMM_MIN_ROWS`,
    :data:`WIDE_GEMM_SHAPES`) and return the threshold. ``min_rows=None`` measures (cached),
    0 disables, N forces N -- still only for the shapes that verify at N (calibrate.py:965-985)."""
    global WIDE_GEMM_MIN_ROWS, WIDE_GEMM_SHAPES
    from .wide_gemm import SAFE_MIN_ROWS, verified_shapes

    if min_rows is None:
        WIDE_GEMM_MIN_ROWS, WIDE_GEMM_SHAPES = wide_gemm_min_rows(target, drafter, target_repo=target_repo,
                                                                  cache_dir=cache_dir, verbose=verbose)
    else:
        WIDE_GEMM_MIN_ROWS = max(int(min_rows), SAFE_MIN_ROWS) if int(min_rows) else None
        WIDE_GEMM_SHAPES = (verified_shapes([getattr(target, "model", target), drafter], WIDE_GEMM_MIN_ROWS)
                            if WIDE_GEMM_MIN_ROWS else [])
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
