"""Pins oracle/moe_ref.py: routing against a brute-force restatement (math.exp softmax,
Python's sorted() over (logit desc, id asc)), deliberate ties, permutation invariance, the
bucketing invariants, the grouped qmm against dequantize-and-matmul per pair, the SwiGLU
closed form, the whole SwitchGLU block against a float64 composition, and the C routing."""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import c_oracle, moe_ref, quant_ref


def _logits(seed, M=16, E=128):
    r = np.random.Generator(np.random.PCG64(seed))
    return quant_ref.bf16_round(r.standard_normal((M, E)).astype(np.float32))


def test_route_matches_brute_force():
    x = _logits(0)
    inds, scores = moe_ref.route(x, 8)
    for t in range(x.shape[0]):
        row = [float(v) for v in x[t]]
        top = sorted(range(len(row)), key=lambda j: (-row[j], j))[:8]
        assert inds[t].tolist() == top
        z = sum(math.exp(v - max(row)) for v in row)
        g = [math.exp(row[j] - max(row)) / z for j in top]
        g = quant_ref.bf16_round(np.array(g, dtype=np.float32)).astype(np.float64)
        want = g / float(quant_ref.bf16_round(np.float32(g.sum())))
        assert np.abs(scores[t] - want).max() <= 2 ** -8 * want.max()
        assert abs(scores[t].sum() - 1.0) < 2e-2


def test_route_ties_and_renorm_off():
    x = np.zeros((2, 16), dtype=np.float32)
    x[1, [3, 9, 12]] = 1.0
    inds, scores = moe_ref.route(x, 4)
    assert inds[0].tolist() == [0, 1, 2, 3]                 # all tied: lowest ids
    assert np.all(scores[0] == 0.25)
    assert inds[1].tolist() == [3, 9, 12, 0]                # tie among the 1.0s by id, then the 0s
    raw_inds, raw = moe_ref.route(x, 4, renorm=False)
    assert np.array_equal(raw_inds, inds)
    assert np.all(raw[0] == quant_ref.bf16_round(np.float32(1 / 16)))


def test_route_permutation_invariance():
    x = _logits(1, M=4, E=32)
    perm = np.random.Generator(np.random.PCG64(2)).permutation(32)
    a, sa = moe_ref.route(x, 6)
    b, sb = moe_ref.route(x[:, perm], 6)
    assert np.array_equal(perm[b], a) and np.array_equal(sa, sb)


def test_bucket_invariants():
    inds, _ = moe_ref.route(_logits(3), 8)
    off, srt, pos = moe_ref.bucket(inds, 128)
    flat = inds.reshape(-1)
    assert off[0] == 0 and off[-1] == flat.size and np.all(np.diff(off) == np.bincount(flat, minlength=128))
    for e in range(128):
        seg = srt[off[e]:off[e + 1]]
        assert np.all(flat[seg] == e) and np.all(np.diff(seg) > 0)      # stable in pair id
    assert np.array_equal(srt[pos], np.arange(flat.size))


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_qmm_matches_dequant_matmul(bits):
    r = np.random.Generator(np.random.PCG64(4))
    E, N, K = 4, 32, 128
    mats = [quant_ref.random_packed(r, N, K, bits) for _ in range(E)]
    w, s, b = (np.stack([m[i] for m in mats]) for i in range(3))
    x = quant_ref.bf16_round(r.standard_normal((3, K)).astype(np.float32))
    rows, experts = [0, 2, 1, 0, 2], [3, 0, 0, 1, 3]
    y = moe_ref.gather_qmm(x, rows, experts, w, s, b, bits)
    for p, (rr, e) in enumerate(zip(rows, experts)):
        ref = x[rr].astype(np.float64) @ quant_ref.dequantize(w[e], s[e], b[e], bits).astype(np.float64).T
        assert np.abs(y[p] - ref).max() <= 2 ** -8 * np.abs(ref).max() + 1e-6


def test_swiglu_closed_form():
    g = np.array([0.0, 1.0, -2.0, 3.5], dtype=np.float32)
    u = np.array([5.0, 1.0, 0.5, -1.0], dtype=np.float32)
    h = moe_ref.swiglu(g, u)
    want = [0.0] + [float(quant_ref.bf16_round(np.float32(
        quant_ref.bf16_round(np.float32(gg * quant_ref.bf16_round(np.float32(1 / (1 + math.exp(-gg)))))) * uu)))
        for gg, uu in zip(g[1:], u[1:])]
    assert h.tolist() == want
    assert abs(h[1] - 1 / (1 + math.exp(-1))) < 2 ** -7


def test_switch_glu_matches_float64_composition():
    r = np.random.Generator(np.random.PCG64(5))
    E, H, I, k, M = 8, 128, 64, 2, 3
    def stack(n, kk):
        mats = [quant_ref.random_packed(r, n, kk, 4) for _ in range(E)]
        return tuple(np.stack([m[i] for m in mats]) for i in range(3))
    gate, up, down = stack(I, H), stack(I, H), stack(H, I)
    x = quant_ref.bf16_round(r.standard_normal((M, H)).astype(np.float32))
    logits = _logits(6, M=M, E=E)
    out, inds, scores = moe_ref.switch_glu(x, logits, *gate, *up, *down, k=k, bits=4)
    deq = lambda t, e: quant_ref.dequantize(t[0][e], t[1][e], t[2][e], 4).astype(np.float64)
    bf = lambda a: quant_ref.bf16_round(np.asarray(a, dtype=np.float32)).astype(np.float64)
    for t in range(M):
        exact = np.zeros(H)            # no intermediate rounding
        same = np.zeros(H)             # mlx's bf16 rounding points, by dequantize-and-matmul
        for j in range(k):
            e = int(inds[t, j])
            gg = x[t] @ deq(gate, e).T
            uu = x[t] @ deq(up, e).T
            exact += scores[t, j] * ((gg / (1 + np.exp(-gg)) * uu) @ deq(down, e).T)
            g2, u2 = bf(gg), bf(uu)
            h2 = bf(bf(g2 * bf(1 / (1 + np.exp(-g2)))) * u2)
            same += bf(scores[t, j] * bf(h2 @ deq(down, e).T))
        assert np.abs(out[t] - bf(same)).max() <= 2 ** -7 * np.abs(same).max()
        # the bf16 rounding points cost a few percent of RMS against unrounded arithmetic
        assert np.abs(out[t] - exact).max() <= 4e-2 * np.sqrt(np.mean(exact ** 2))


def test_c_route_matches_numpy():
    x = _logits(7, M=16, E=128)
    x[3, [5, 77]] = 9.0                                       # a tie at the top
    ci, cs = c_oracle.route(quant_ref.bf16_bits(x), 8)
    ni, ns = moe_ref.route(x, 8)
    assert np.array_equal(ci, ni)
    assert np.array_equal(quant_ref.bf16_round(np.asarray(cs, dtype=np.float32)), ns)
