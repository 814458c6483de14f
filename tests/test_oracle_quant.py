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


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_rule_kats(bits):
    """The quantizer's rule at its fixed points: bias = bf16(min), scale = bf16((max - min) /
    (2^bits - 1)); the group minimum maps to field 0, the maximum to round((max - min) / scale)
    (the top field unless the scale's bf16 rounding went up); a constant group has scale 0
    (fields 0, bias = the value); a midpoint rounds half to even."""
    levels = (1 << bits) - 1
    w = np.zeros((3, 64), np.float32)
    w[0] = np.linspace(-1.0, 2.0, 64, dtype=np.float32)
    w[1] = 0.75
    w[2, :32], w[2, 32:] = -0.5, 0.5
    q, s, b = quant_ref.quantize(w, bits)
    f = quant_ref.unpack(q, bits)
    assert b[0, 0] == -1.0 and s[0, 0] == quant_ref.bf16_round(np.float32(3.0 / levels))
    assert f[0, 0] == 0 and f[0, -1] == levels
    assert s[1, 0] == 0.0 and b[1, 0] == 0.75 and not f[1].any()
    # range 1.0: scale = bf16(1/levels) rounds up (1/255 -> 0x3B81 = 0.0039367676, 1/15 ->
    # 0x3D89 = 0.0668945), so the top value lands at round(1 / scale): 254 at 8 bits, 15 at 4
    top = {8: 254, 4: 15}[bits]
    assert s[2, 0] == {8: 0.003936767578125, 4: 0.06689453125}[bits]
    assert b[2, 0] == -0.5 and set(f[2].tolist()) == {0, top}
    # a value exactly halfway between two fields takes the even one
    half = np.zeros((1, 64), np.float32)
    half[0, 1] = 1.0                         # scale 1/levels, bias 0
    sc = float(quant_ref.quantize(half, bits)[1][0, 0])
    half[0, 2] = np.float32(2.5 * sc)        # 2.5 steps above the bias
    f2 = quant_ref.unpack(quant_ref.quantize(half, bits)[0], bits)
    assert f2[0, 2] == 2
