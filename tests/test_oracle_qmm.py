"""CPU: the qmm oracle pinned by independent computations (not by retyping its formula).

* dequantize-then-matmul (a different evaluation order: distributivity of the factored form)
* scales = 1, biases = 0: exact integer arithmetic
* one-hot x: a dequantized column
* a pure-Python loop over the definition at K = 64, N = 8
* linearity in x, row-count invariance, the C restatement
"""

from __future__ import annotations

import numpy as np
import pytest

from _util import randn_bf16, rng
from oracle import c_oracle, qmm_ref, quant_ref


def _mats(seed, n, k, bits):
    r = rng(seed)
    return r, quant_ref.random_packed(r, n, k, bits)


@pytest.mark.parametrize("bits", [4, 8])
def test_factored_equals_dequant_matmul(bits):
    r, (w, s, b) = _mats(1, 32, 256, bits)
    x = randn_bf16(r, 5, 256)
    y = qmm_ref.qmm_f64(x, w, s, b, bits)
    ref = x.astype(np.float64) @ quant_ref.dequantize(w, s, b, bits).T
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("bits", [4, 8])
def test_unit_scale_zero_bias_is_integer_matmul(bits):
    r = rng(2)
    q = r.integers(0, 1 << bits, size=(8, 128))
    w = quant_ref.pack(q, bits)
    s = np.ones((8, 2), np.float32)
    b = np.zeros((8, 2), np.float32)
    xi = r.integers(-8, 9, size=(3, 128))
    y = qmm_ref.qmm_f64(xi.astype(np.float32), w, s, b, bits)
    assert np.array_equal(y, (xi @ q.T).astype(np.float64))


@pytest.mark.parametrize("bits", [4, 8])
def test_one_hot_selects_dequantized_column(bits):
    r, (w, s, b) = _mats(3, 16, 128, bits)
    j = 77
    x = np.zeros((1, 128), np.float32)
    x[0, j] = 1.0
    y = qmm_ref.qmm_f64(x, w, s, b, bits)[0]
    qcol = quant_ref.unpack(w, bits)[:, j]
    assert np.allclose(y, s[:, j // 64] * qcol + b[:, j // 64], rtol=0, atol=1e-12)


@pytest.mark.parametrize("bits", [4, 8])
def test_pure_python_definition(bits):
    r, (w, s, b) = _mats(4, 8, 64, bits)
    x = randn_bf16(r, 2, 64)
    f = 32 // bits
    ref = np.zeros((2, 8))
    for m in range(2):
        for n in range(8):
            acc = 0.0
            for j in range(64):
                word = int(w[n, j // f])
                qv = (word >> (bits * (j % f))) & ((1 << bits) - 1)
                acc += float(x[m, j]) * (float(s[n, 0]) * qv + float(b[n, 0]))
            ref[m, n] = acc
    assert np.allclose(qmm_ref.qmm_f64(x, w, s, b, bits), ref, rtol=1e-12, atol=1e-12)


def test_linearity_and_row_invariance():
    r, (w, s, b) = _mats(5, 24, 192, 4)
    x1, x2 = randn_bf16(r, 4, 192), randn_bf16(r, 4, 192)
    y = qmm_ref.qmm_f64
    assert np.allclose(y(x1 + x2, w, s, b, 4), y(x1, w, s, b, 4) + y(x2, w, s, b, 4), atol=1e-10)
    assert np.allclose(y(3.0 * x1, w, s, b, 4), 3.0 * y(x1, w, s, b, 4), atol=1e-10)
    full = y(x1, w, s, b, 4)
    assert np.array_equal(full[:2], y(x1[:2], w, s, b, 4))


@pytest.mark.parametrize("bits", [4, 8])
def test_c_restatement_matches(bits):
    r, (w, s, b) = _mats(6, 64, 512, bits)
    x = randn_bf16(r, 16, 512)
    yc = c_oracle.qmm(quant_ref.bf16_bits(x), w, quant_ref.bf16_bits(s), quant_ref.bf16_bits(b), bits)
    y = qmm_ref.qmm_f64(x, w, s, b, bits)
    assert np.max(np.abs(yc - y)) <= 1e-5 * max(1.0, np.abs(y).max())


def test_rms_tolerance_helper():
    ok, err, r = qmm_ref.within_rms_tol(np.array([1.0, 1.0]), np.array([1.0, 1.01]))
    assert ok and err == pytest.approx(0.01) and r > 1.0
    ok, _, _ = qmm_ref.within_rms_tol(np.array([1.0, 2.0]), np.array([1.0, 1.0]))
    assert not ok
