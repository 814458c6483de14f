"""Pins oracle/attn_ref.py: the exact attention definition against a pure-Python per-element
loop, GQA against tiled MHA, row independence, the causal leak KAT
(tests/test_multirow_attn.py:90-99), uniform keys, the tree mask's special cases, the multirow
restatement against the exact form and across block splits, the row split
(sdpa_split.py:61-93), and the C restatement."""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import attn_ref, c_oracle, quant_ref


def _mk(seed, B=1, hq=4, hk=2, mq=3, L=11, d=8, dtype=np.float64):
    r = np.random.Generator(np.random.PCG64(seed))
    q = r.standard_normal((B, hq, mq, d)).astype(dtype)
    k = r.standard_normal((B, hk, L, d)).astype(dtype)
    v = r.standard_normal((B, hk, L, d)).astype(dtype)
    return q, k, v


def _python_attention(q, k, v, scale, causal):
    B, hq, mq, d = q.shape
    hk, L = k.shape[1], k.shape[2]
    out = np.zeros_like(q)
    for b in range(B):
        for h in range(hq):
            kv = h // (hq // hk)
            for i in range(mq):
                last = (L - mq + i) if causal else (L - 1)        # keys 0..last are visible
                s = [sum(q[b, h, i, t] * k[b, kv, j, t] for t in range(d)) * scale for j in range(last + 1)]
                mx = max(s)
                e = [math.exp(x - mx) for x in s]
                z = sum(e)
                for t in range(d):
                    out[b, h, i, t] = sum(e[j] * v[b, kv, j, t] for j in range(last + 1)) / z
    return out


@pytest.mark.parametrize("causal", [True, False])
def test_exact_form_matches_python_loop(causal):
    q, k, v = _mk(0, B=2)
    got = attn_ref.attention(q, k, v, 0.3, causal)
    assert np.abs(got - _python_attention(q, k, v, 0.3, causal)).max() < 1e-12


def test_gqa_equals_tiled_mha():
    q, k, v = _mk(1, hq=6, hk=2)
    kt, vt = np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1)
    assert np.abs(attn_ref.attention(q, k, v, 0.25) - attn_ref.attention(q, kt, vt, 0.25)).max() < 1e-14


def test_row_independence():
    q, k, v = _mk(2, mq=5, L=20)
    full = attn_ref.attention(q, k, v, 0.2, causal=True)
    for i in range(5):
        end = 20 - 5 + i + 1
        one = attn_ref.attention(q[:, :, i:i + 1], k[:, :, :end], v[:, :, :end], 0.2, causal=False)
        assert np.abs(full[:, :, i:i + 1] - one).max() < 1e-13


def test_causal_leak_kat():
    """Masked keys made dominant (50) with huge values (1e3): a leak would swamp the rows."""
    q, k, v = _mk(3, hq=4, hk=4, mq=4, L=64, d=64)
    k[:, :, -3:] = 50.0
    v[:, :, -3:] = 1e3
    out = attn_ref.attention(q, k, v, 0.125, causal=True)
    assert np.abs(out[:, :, 0]).max() < 10.0           # row 0 sees none of the last 3 keys
    assert np.abs(out[:, :, 3]).max() > 500.0          # the last row sees them and is dominated


def test_uniform_keys_average_values():
    q, k, v = _mk(4, mq=4, L=9)
    k[:] = 0.0
    out = attn_ref.attention(q, k, v, 1.0, causal=True)
    for i in range(4):
        vis = 9 - 4 + i + 1
        assert np.allclose(out[:, :, i], np.repeat(v[:, :, :vis].mean(axis=2), 2, axis=1), atol=1e-14)


def test_tree_mask_special_cases():
    q, k, v = _mk(5, mq=4, L=10)
    lower = [(1 << (i + 1)) - 1 for i in range(4)]              # ancestors = all earlier rows
    assert np.abs(attn_ref.attention(q, k, v, 0.3, tree_anc=lower) - attn_ref.attention(q, k, v, 0.3)).max() < 1e-14
    m = attn_ref.visible_mask(4, 10, tree_anc=[1, 2, 4, 8])        # self only
    assert m[:, :6].all() and np.array_equal(m[:, 6:], np.eye(4, dtype=bool))
    assert np.array_equal(attn_ref.visible_mask(3, 5, causal=True),
                          np.array([[1, 1, 1, 0, 0], [1, 1, 1, 1, 0], [1, 1, 1, 1, 1]], dtype=bool))


def test_multirow_restatement_close_to_exact_and_split_invariant():
    q, k, v = _mk(6, hq=8, hk=2, mq=8, L=300, d=64, dtype=np.float32)
    q, k, v = (quant_ref.bf16_round(t) for t in (q, k, v))
    exact = attn_ref.attention(q, k, v, 64 ** -0.5, causal=True)
    rms = np.sqrt(np.mean(exact ** 2))
    outs = [attn_ref.attention_multirow(q, k, v, 64 ** -0.5, causal=True, chunk=c) for c in (None, 64, 96)]
    for o in outs:
        assert np.abs(o - exact).max() <= 2e-2 * rms
    assert np.abs(outs[0] - outs[1]).max() <= 2 ** -7 * np.abs(exact).max()   # bf16 output ulps
    tree = [(1 << (i + 1)) - 1 if i % 2 else 1 << i for i in range(8)]
    t_exact = attn_ref.attention(q, k, v, 64 ** -0.5, causal=False, tree_anc=tree)
    t_mr = attn_ref.attention_multirow(q, k, v, 64 ** -0.5, causal=False, tree_anc=tree, chunk=64)
    assert np.abs(t_mr - t_exact).max() <= 2e-2 * np.sqrt(np.mean(t_exact ** 2))


def test_split_sdpa_is_exact_and_partition_kats():
    q, k, v = _mk(7, mq=12, L=40)
    full = attn_ref.attention(q, k, v, 0.2, causal=True)
    for mc in (1, 3, 5, 12):
        assert np.abs(attn_ref.split_sdpa(q, k, v, 0.2, True, mc) - full).max() < 1e-13
    assert np.abs(attn_ref.split_sdpa(q, k, v, 0.2, False, 5) - attn_ref.attention(q, k, v, 0.2, False)).max() < 1e-13
    assert attn_ref.partition(12, 5) == [4, 4, 4]
    assert attn_ref.partition(11, 5) == [4, 4, 3]
    assert attn_ref.partition(3, 5) == [3]


@pytest.mark.parametrize("tree", [False, True])
def test_c_restatement_matches(tree):
    q, k, v = _mk(8, hq=8, hk=2, mq=6, L=200, d=64, dtype=np.float32)
    q, k, v = (quant_ref.bf16_round(t) for t in (q, k, v))
    anc = [(1 << (i + 1)) - 1 if i % 2 else 1 << i for i in range(6)] if tree else None
    exact = attn_ref.attention(q, k, v, 0.125, causal=not tree, tree_anc=anc)
    got = c_oracle.attention(quant_ref.bf16_bits(q), quant_ref.bf16_bits(k), quant_ref.bf16_bits(v), 0.125,
                             causal=not tree, tree_anc=anc)
    assert np.abs(got - exact).max() <= 2e-2 * np.sqrt(np.mean(exact ** 2))


def test_quantized_kv_oracle_pins():
    """dequantize_kv is the affine format row by row: unit scales and zero biases give the
    integer fields themselves (an integer-valued cache, attended exactly like plain K/V);
    general scales/biases match the per-row dequantize of quant_ref; attention_quantized is
    attention over those values."""
    from oracle import quant_ref

    r = np.random.Generator(np.random.PCG64(9))
    for bits in (4, 8):
        B, H, L, D = 1, 2, 37, 128
        ints = r.integers(0, 1 << bits, (B * H * L, D))
        words = quant_ref.pack(ints, bits).reshape(B, H, L, D * bits // 32)
        ones = np.ones((B, H, L, D // 64), np.float32)
        zeros = np.zeros_like(ones)
        assert np.array_equal(attn_ref.dequantize_kv(words, ones, zeros, bits), ints.reshape(B, H, L, D))
        s = quant_ref.bf16_round(r.uniform(0.01, 0.1, (B, H, L, D // 64)).astype(np.float32))
        b = quant_ref.bf16_round(r.normal(0, 0.5, (B, H, L, D // 64)).astype(np.float32))
        got = attn_ref.dequantize_kv(words, s, b, bits)
        want = ints.reshape(B, H, L, 2, 64) * s[..., None].astype(np.float64) + b[..., None]
        assert np.allclose(got, want.reshape(B, H, L, D), rtol=0, atol=0)
        q = r.standard_normal((B, 4, 5, D))
        vals = (words, s, b)
        plain = attn_ref.attention(q, got, got, 0.1, causal=True)
        assert np.array_equal(attn_ref.attention_quantized(q, vals, vals, 0.1, bits, causal=True), plain)
