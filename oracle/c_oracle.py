"""ctypes wrapper of oracle/_build/liboracle.so (the C/OpenMP restatement in dspark_oracle.c).

Test infrastructure: numpy in, numpy out. Built by ``make -C oracle`` (also by
``__graft_entry__.build()``).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "liboracle.so")
_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64


def build() -> str:
    subprocess.run(["make", "-B", "-s", "-C", HERE], check=True)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        lib = ctypes.CDLL(LIB)
        lib.orc_threads.restype = ctypes.c_int
        lib.orc_set_threads.argtypes = [ctypes.c_int]
        lib.orc_qmm.argtypes = [_p, _i64, _i64, _p, _p, _p, _i64, ctypes.c_int, _p]
        lib.orc_attention.argtypes = [_p, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _i64, ctypes.c_float,
                                      ctypes.c_int, _p, _p]
        lib.orc_route.argtypes = [_p, _i64, _i64, _i64, ctypes.c_int, _p, _p]
        lib.orc_unpack.argtypes = [_p, _i64, ctypes.c_int, _p]
        _lib = lib
    return _lib


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def threads() -> int:
    return int(load().orc_threads())


def set_threads(n: int) -> None:
    load().orc_set_threads(int(n))


def unpack(w: np.ndarray, bits: int) -> np.ndarray:
    w = _c(w, np.uint32)
    q = np.empty((w.shape[0], w.shape[1] * 32 // bits), dtype=np.int32)
    load().orc_unpack(w.ctypes.data, w.size, bits, q.ctypes.data)
    return q


def qmm(x_bits: np.ndarray, w: np.ndarray, s_bits: np.ndarray, b_bits: np.ndarray, bits: int) -> np.ndarray:
    """x/scales/biases as bf16 bit patterns (uint16); returns fp32 [M, N] before bf16 rounding."""
    x_bits = _c(x_bits, np.uint16)
    w = _c(w, np.uint32)
    s_bits = _c(s_bits, np.uint16)
    b_bits = _c(b_bits, np.uint16)
    m, k = x_bits.shape
    n = w.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    load().orc_qmm(x_bits.ctypes.data, m, k, w.ctypes.data, s_bits.ctypes.data, b_bits.ctypes.data, n, bits,
                   y.ctypes.data)
    return y


def attention(q_bits, k_bits, v_bits, scale: float, causal: bool = True, tree_anc=None) -> np.ndarray:
    """q [B,Hq,Mq,D], k/v [B,Hk,L,D] as bf16 bit patterns (contiguous); fp32 output."""
    q_bits = _c(q_bits, np.uint16)
    k_bits = _c(k_bits, np.uint16)
    v_bits = _c(v_bits, np.uint16)
    B, Hq, Mq, D = q_bits.shape
    Hk, L = k_bits.shape[1], k_bits.shape[2]
    ks = np.array([Hk * L * D, L * D, D], dtype=np.int64)
    out = np.empty((B, Hq, Mq, D), dtype=np.float32)
    anc = None if tree_anc is None else _c(tree_anc, np.uint32)
    load().orc_attention(q_bits.ctypes.data, B, Hq, Mq, D, k_bits.ctypes.data, v_bits.ctypes.data, ks.ctypes.data,
                         ks.ctypes.data, Hk, L, float(scale), int(bool(causal)),
                         None if anc is None else anc.ctypes.data, out.ctypes.data)
    return out


def route(logits_bits: np.ndarray, k: int, renorm: bool = True):
    logits_bits = _c(logits_bits, np.uint16)
    M, E = logits_bits.shape
    inds = np.empty((M, k), dtype=np.int32)
    scores = np.empty((M, k), dtype=np.float32)
    load().orc_route(logits_bits.ctypes.data, M, E, k, int(bool(renorm)), inds.ctypes.data, scores.ctypes.data)
    return inds, scores
