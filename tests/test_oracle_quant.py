"""CPU: the packed affine format (oracle/quant_ref.py) pinned by hand KATs, round trips, a
pure-Python bit loop, and the C restatement; plus the product quantizer's torch helpers."""

from __future__ import annotations

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from _util import rng
from oracle import c_oracle, quant_ref


def test_unpack_kats():
    # reference layout (skinny_qmm.py:95-119): field f of a word holds element f, low bits first
    assert quant_ref.unpack(np.array([[0x76543210]], dtype=np.uint32), 4).tolist() == [[0, 1, 2, 3, 4, 5, 6, 7]]
    assert quant_ref.unpack(np.array([[0x04030201]], dtype=np.uint32), 8).tolist() == [[1, 2, 3, 4]]
    assert quant_ref.unpack(np.array([[0xFEDCBA98]], dtype=np.uint32), 4).tolist() == [[8, 9, 10, 11, 12, 13, 14, 15]]
    assert quant_ref.unpack(np.array([[0xFF00807F]], dtype=np.uint32), 8).tolist() == [[0x7F, 0x80, 0x00, 0xFF]]


def _bitloop_unpack(word: int, bits: int) -> list[int]:
    out, mask = [], (1 << bits) - 1
    for f in range(32 // bits):
        out.append((word >> (bits * f)) & mask)
    return out


@pytest.mark.parametrize("bits", [4, 8])
def test_unpack_matches_bit_loop(bits):
    r = rng(1)
    w = r.integers(0, 2**32, size=(3, 17), dtype=np.uint64).astype(np.uint32)
    got = quant_ref.unpack(w, bits)
    ref = [[v for word in row for v in _bitloop_unpack(int(word), bits)] for row in w]
    assert got.tolist() == ref


@settings(max_examples=40, deadline=None)
@given(bits=st.sampled_from([4, 8]), n=st.integers(1, 5), words=st.integers(1, 6), seed=st.integers(0, 2**31))
def test_pack_unpack_round_trip(bits, n, words, seed):
    r = rng(seed)
    k = words * 32 // bits
    q = r.integers(0, 1 << bits, size=(n, k))
    assert np.array_equal(quant_ref.unpack(quant_ref.pack(q, bits), bits), q)


@pytest.mark.parametrize("bits", [4, 8])
def test_c_unpack_matches_numpy(bits):
    r = rng(2)
    w = r.integers(0, 2**32, size=(5, 24), dtype=np.uint64).astype(np.uint32)
    assert np.array_equal(c_oracle.unpack(w, bits), quant_ref.unpack(w, bits))


def test_bf16_rounding_kats():
    # ties to even at the bf16 boundary; exact values untouched
    vals = np.array([1.0, 1.00390625, 1.01171875, -2.5, 3.0e38], dtype=np.float32)
    out = quant_ref.bf16_round(vals)
    assert out[0] == 1.0
    assert out[1] == 1.0            # 1 + 2^-8 is a tie -> even (1.0)
    assert out[2] == 1.015625       # 1 + 3*2^-8 is a tie -> even (1 + 2^-6)
    assert out[3] == -2.5
    bits = quant_ref.bf16_bits(np.array([1.0, -2.0], dtype=np.float32))
    assert bits.tolist() == [0x3F80, 0xC000]


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_dequantize_error_bound(bits):
    r = rng(3)
    w = (r.standard_normal((8, 256)) * 0.02).astype(np.float32)
    wq, s, b = quant_ref.quantize(w, bits)
    deq = quant_ref.dequantize(wq, s, b, bits)
    # round-to-nearest over [min, max]: error <= scale/2 (+ bf16 rounding of scale/bias)
    step = np.repeat(s, 64, axis=1)
    assert np.all(np.abs(deq - w) <= 0.5 * step + 2e-3 * np.abs(w).max())


def test_torch_quant_matches_oracle():
    import sys

    torch = pytest.importorskip("torch")
    from dspark_rocm import quant

    r = rng(4)
    for bits in (4, 8):
        q = r.integers(0, 1 << bits, size=(6, 128))
        packed = quant.pack(torch.from_numpy(q), bits)
        ref = quant_ref.pack(q, bits).view(np.int32)
        assert np.array_equal(packed.numpy(), ref)
        assert np.array_equal(quant.unpack(packed, bits).numpy(), q)
        w = torch.from_numpy((r.standard_normal((4, 128)) * 0.02).astype(np.float32))
        pw, s, b = quant.quantize(w, bits=bits)
        deq = quant.dequantize(pw, s, b, bits=bits)
        assert float((deq - w).abs().max()) <= float(s.float().max()) * 0.5 + 1e-3
    assert "dspark_rocm" in sys.modules
