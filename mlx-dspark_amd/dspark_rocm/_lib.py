"""ctypes binding of the gfx950 kernel library (``libdspark_rocm.so``, C ABI in include/dspark.h).

The library is built in-tree by ``mlx-dspark_amd/build.py``. There is no fallback: if the
library is missing or fails to load, every kernel entry point raises :class:`DsparkUnavailable`.
A non-zero status from a kernel call raises :class:`DsparkError` carrying the library's message
(the reference's kernels raise on a refused launch, skinny_qmm.py:207-211).
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdspark_rocm.so")

c_void_p = ctypes.c_void_p
c_int = ctypes.c_int
c_i64 = ctypes.c_int64
c_size_t = ctypes.c_size_t
c_float = ctypes.c_float
c_char_p = ctypes.c_char_p
c_i64_p = ctypes.POINTER(ctypes.c_int64)

STATUS = {
    0: "DSPARK_OK",
    -1: "DSPARK_ERR_ARG",
    -2: "DSPARK_ERR_SHAPE",
    -3: "DSPARK_ERR_ALIGN",
    -4: "DSPARK_ERR_WORKSPACE",
    -5: "DSPARK_ERR_LAUNCH",
    -6: "DSPARK_ERR_UNSUPPORTED",
}


class DsparkUnavailable(RuntimeError):
    """The HIP kernel library is not built or cannot be loaded."""


class DsparkError(RuntimeError):
    """A kernel entry point returned a non-zero dspark_status."""

    def __init__(self, fn: str, status: int, message: str):
        self.fn, self.status, self.message = fn, status, message
        super().__init__(f"{fn}: {STATUS.get(status, status)}: {message}")


class QmmProblem(ctypes.Structure):
    """``dspark_qmm_problem`` (include/dspark.h)."""

    _fields_ = [
        ("x", c_void_p),
        ("ldx", c_i64),
        ("w", c_void_p),
        ("scales", c_void_p),
        ("biases", c_void_p),
        ("y", c_void_p),
        ("ldy", c_i64),
        ("N", c_i64),
        ("K", c_i64),
    ]


class QmmPackedProblem(ctypes.Structure):
    """``dspark_qmm_packed_problem`` (include/dspark.h)."""

    _fields_ = [
        ("x", c_void_p),
        ("ldx", c_i64),
        ("packed", c_void_p),
        ("y", c_void_p),
        ("ldy", c_i64),
        ("N", c_i64),
        ("K", c_i64),
    ]


MAX_QMM_PROBLEMS = 4

# name -> (restype, argtypes). Every symbol include/dspark.h declares.
SIGNATURES: dict[str, tuple] = {
    "dspark_version": (c_char_p, []),
    "dspark_last_error": (c_char_p, []),
    "dspark_qmm_affine": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_void_p, c_i64,
                                  c_int, c_int, c_void_p, c_i64, c_void_p, c_size_t, c_void_p]),
    "dspark_qmm_affine_workspace": (c_size_t, [c_i64, c_i64, c_i64, c_int, c_int]),
    "dspark_qmm_workspace_reset": (c_int, [c_void_p, c_size_t, c_void_p]),
    "dspark_stream_read": (c_int, [c_void_p, c_size_t, c_void_p, c_void_p]),
    "dspark_qmm_dequantize": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_i64, c_i64, c_int, c_int, c_int,
                                      c_void_p, c_i64, c_void_p]),
    "dspark_qmm_affine_noalloc": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_void_p, c_i64,
                                          c_int, c_int, c_void_p, c_i64, c_void_p]),
    "dspark_qmm_noalloc_reset": (c_int, [c_void_p]),
    "dspark_qmm_noalloc_scratch": (c_int, [ctypes.POINTER(c_void_p), ctypes.POINTER(c_size_t)]),
    "dspark_qmm_affine_supported": (c_int, [c_i64, c_i64, c_i64, c_int, c_int]),
    "dspark_qmm_affine_plan": (c_int, [c_i64, c_i64, c_i64, c_int, c_int, ctypes.POINTER(ctypes.c_int32)]),
    "dspark_qmm_affine_multi": (c_int, [ctypes.POINTER(QmmProblem), c_int, c_i64, c_int, c_int, c_void_p,
                                        c_size_t, c_void_p]),
    "dspark_qmm_affine_multi_workspace": (c_size_t, [ctypes.POINTER(QmmProblem), c_int, c_i64, c_int, c_int]),
    "dspark_qmm_packed_bytes": (c_size_t, [c_i64, c_i64, c_int, c_int]),
    "dspark_qmm_pack": (c_int, [c_void_p, c_void_p, c_void_p, c_i64, c_i64, c_int, c_int, c_void_p, c_size_t,
                                c_void_p]),
    "dspark_qmm_packed_multi": (c_int, [ctypes.POINTER(QmmPackedProblem), c_int, c_i64, c_int, c_int, c_void_p,
                                        c_size_t, c_void_p]),
    "dspark_qmm_packed_multi_workspace": (c_size_t, [ctypes.POINTER(QmmPackedProblem), c_int, c_i64, c_int,
                                                     c_int]),
    "dspark_qmm_packed_multi_plan": (c_int, [ctypes.POINTER(QmmPackedProblem), c_int, c_i64, c_int, c_int,
                                             ctypes.POINTER(ctypes.c_int32)]),
    "dspark_qmm_swiglu_packed_bytes": (c_size_t, [c_i64, c_i64, c_int, c_int]),
    "dspark_qmm_pack_swiglu": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_i64, c_i64,
                                       c_int, c_int, c_void_p, c_size_t, c_void_p]),
    "dspark_qmm_swiglu_packed": (c_int, [c_void_p, c_i64, c_void_p, c_void_p, c_i64, c_i64, c_i64, c_i64, c_int,
                                         c_int, c_void_p, c_size_t, c_void_p]),
    "dspark_qmm_swiglu_packed_workspace": (c_size_t, [c_i64, c_i64, c_i64, c_int, c_int]),
    "dspark_verify_attention": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_i64_p,
                                        c_i64_p, c_i64, c_i64, c_float, c_int, c_void_p, c_void_p, c_void_p,
                                        c_size_t, c_void_p]),
    "dspark_verify_attention_strided": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_i64_p,
                                                c_i64_p, c_i64, c_i64, c_float, c_int, c_void_p, c_void_p, c_i64_p,
                                                c_void_p, c_size_t, c_void_p]),
    "dspark_verify_attention_typed": (c_int, [c_int, c_void_p, c_i64, c_i64, c_i64, c_i64, c_void_p, c_void_p,
                                              c_i64_p, c_i64_p, c_i64, c_i64, c_float, c_int, c_void_p, c_void_p,
                                              c_i64_p, c_void_p, c_size_t, c_void_p]),
    "dspark_verify_attention_quantized": (c_int, [c_int, c_void_p, c_i64, c_i64, c_i64, c_i64,
                                                  c_void_p, c_void_p, c_void_p, c_i64_p, c_i64_p,
                                                  c_void_p, c_void_p, c_void_p, c_i64_p, c_i64_p,
                                                  c_i64, c_i64, c_float, c_int, c_int, c_int, c_void_p, c_i64_p,
                                                  c_void_p, c_size_t, c_void_p]),
    "dspark_verify_attention_workspace": (c_size_t, [c_i64, c_i64, c_i64, c_i64, c_i64, c_i64]),
    "dspark_verify_attention_blocks": (c_i64, [c_i64, c_i64, c_i64, c_i64, c_i64, c_i64]),
    "dspark_verify_attention_plan": (c_int, [c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                             ctypes.POINTER(ctypes.c_int32)]),
    "dspark_moe_route_topk": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_int, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p]),
    "dspark_gather_qmm": (c_int, [c_void_p, c_i64, c_i64, c_void_p, c_void_p, c_i64, c_i64, c_void_p,
                                  c_void_p, c_void_p, c_i64, c_int, c_int, c_void_p, c_i64, c_void_p]),
    "dspark_moe_switch_glu": (c_int, [c_void_p, c_void_p, c_i64, c_i64, c_i64, c_i64, c_i64, c_int,
                                      c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_size_t, c_void_p]),
    "dspark_moe_workspace": (c_size_t, [c_i64, c_i64, c_i64, c_i64, c_i64]),
    "dspark_moe_packed_bytes": (c_size_t, [c_i64, c_i64, c_i64, c_int, c_int]),
    "dspark_moe_pack": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_int, c_int, c_void_p, c_size_t, c_void_p]),
    "dspark_moe_switch_glu_packed": (c_int, [c_void_p, c_void_p, c_i64, c_i64, c_i64, c_i64, c_i64, c_int,
                                             c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                             c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p,
                                             c_void_p, c_void_p, c_size_t, c_void_p]),
    "dspark_moe_packed_plan": (c_int, [c_i64, c_i64, c_i64, c_i64, c_i64, c_int, ctypes.POINTER(ctypes.c_int32)]),
    "dspark_rmsnorm": (c_int, [c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64, c_i64, c_float, c_void_p, c_i64,
                               c_void_p, c_i64, c_void_p]),
    "dspark_qk_norm_rope_kv": (c_int, [c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64, c_i64, c_i64, c_i64, c_i64,
                                       c_void_p, c_void_p, c_float, c_float, c_i64, c_void_p, c_void_p, c_i64_p,
                                       c_void_p, c_i64_p, c_void_p]),
    "dspark_qk_norm_rope_kv_quantized": (c_int, [c_void_p, c_i64, c_void_p, c_i64, c_void_p, c_i64, c_i64, c_i64,
                                                 c_i64, c_i64, c_void_p, c_void_p, c_float, c_float, c_i64,
                                                 c_void_p, c_void_p, c_void_p, c_void_p, c_i64_p, c_i64_p,
                                                 c_void_p, c_void_p, c_void_p, c_i64_p, c_i64_p, c_int, c_int,
                                                 c_void_p]),
    "dspark_swiglu": (c_int, [c_void_p, c_i64, c_void_p, c_i64, c_i64, c_i64, c_void_p, c_i64, c_void_p]),
    "dspark_argmax_rows": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_void_p, c_void_p]),
    "dspark_greedy_accept": (c_int, [c_void_p, c_i64, c_void_p, c_void_p, c_void_p]),
    "dspark_argmax_accept_workspace": (c_size_t, [c_i64, c_i64]),
    "dspark_argmax_accept": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_void_p, c_i64, c_void_p, c_void_p, c_void_p,
                                     c_size_t, c_void_p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library once and bind every declared entry point (missing symbol = error)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise DsparkUnavailable(
                f"{path} is not built; run `python mlx-dspark_amd/build.py` (hipcc, gfx950)")
        try:
            lib = ctypes.CDLL(path)
        except OSError as e:  # pragma: no cover - depends on the machine
            raise DsparkUnavailable(f"cannot load {path}: {e}") from e
        missing = []
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError:
                missing.append(name)
                continue
            fn.restype = res
            fn.argtypes = args
        if missing:
            raise DsparkUnavailable(f"{path} lacks {missing}; rebuild it")
        _lib = lib
    return _lib


def exported_symbols(path: str = LIB_PATH) -> list[str]:
    """Names from :data:`SIGNATURES` that the library at ``path`` exports (no kernel calls)."""
    lib = ctypes.CDLL(path)
    return [n for n in SIGNATURES if hasattr(lib, n)]


def available() -> bool:
    try:
        load()
        return True
    except DsparkUnavailable:
        return False


def last_error() -> str:
    return (load().dspark_last_error() or b"").decode()


def check(fn: str, status: int) -> None:
    if status != 0:
        raise DsparkError(fn, int(status), last_error())


def call(name: str, *args) -> int:
    """Call ``name`` and raise :class:`DsparkError` on a non-zero status."""
    st = getattr(load(), name)(*args)
    check(name, st)
    return st
