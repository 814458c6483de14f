"""CPU: the committed golden fixtures (tests/golden/, written by make_golden.py) are reproduced
by the oracle restatements and the C restatement, so a change to either shows up here."""

from __future__ import annotations

import os

import numpy as np

from oracle import attn_ref, c_oracle, moe_ref, qmm_ref, quant_ref, verify_ref

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, f"{name}.npz"))


def test_unpack_fixture():
    f = _load("unpack")
    assert np.array_equal(quant_ref.unpack(f["kat4_word"].reshape(1, 1), 4)[0], f["kat4_vals"])
    assert np.array_equal(quant_ref.unpack(f["kat8_word"].reshape(1, 1), 8)[0], f["kat8_vals"])
    for bits in (4, 8):
        assert np.array_equal(quant_ref.pack(f[f"q{bits}"], bits), f[f"w{bits}"])
        assert np.array_equal(quant_ref.unpack(f[f"w{bits}"], bits), f[f"q{bits}"])
        assert np.array_equal(c_oracle.unpack(f[f"w{bits}"], bits), f[f"q{bits}"])


def test_qmm_fixture():
    f = _load("qmm")
    for bits in (4, 8):
        w, s, b = f[f"w{bits}"], quant_ref.bf16_from_bits(f[f"s{bits}"]), quant_ref.bf16_from_bits(f[f"b{bits}"])
        for m in (1, 5, 8, 16):
            x = quant_ref.bf16_from_bits(f[f"x{bits}_{m}"])
            assert np.array_equal(qmm_ref.qmm_f64(x, w, s, b, bits), f[f"y{bits}_{m}"])
            c = c_oracle.qmm(f[f"x{bits}_{m}"], w, f[f"s{bits}"], f[f"b{bits}"], bits)
            assert qmm_ref.within_rms_tol(c, f[f"y{bits}_{m}"], 1e-3)[0]


def test_attention_fixture():
    f = _load("attention")
    anc = f["tree_anc"]
    for L in (48, 300):
        q, k, v = (quant_ref.bf16_from_bits(f[f"{t}{L}"]) for t in "qkv")
        assert np.array_equal(attn_ref.attention(q, k, v, 128 ** -0.5, causal=True), f[f"causal{L}"])
        assert np.array_equal(attn_ref.attention(q, k, v, 128 ** -0.5, causal=False, tree_anc=anc), f[f"tree{L}"])
        c = c_oracle.attention(f[f"q{L}"], f[f"k{L}"], f[f"v{L}"], 128 ** -0.5, causal=True)
        ref = f[f"causal{L}"]
        assert np.abs(c - ref).max() <= 2e-2 * np.sqrt(np.mean(ref ** 2))


def test_route_fixture():
    f = _load("route")
    x = quant_ref.bf16_from_bits(f["logits"])
    inds, scores = moe_ref.route(x, 8)
    assert np.array_equal(inds, f["inds"]) and np.array_equal(quant_ref.bf16_bits(scores), f["scores"])
    assert f["inds"][2, :3].tolist() == [7, 90, 100] and f["inds"][5].tolist() == list(range(8))
    assert 3 not in f["inds"][9] and 4 not in f["inds"][9]
    off, srt, pos = moe_ref.bucket(inds, 128)
    assert np.array_equal(off, f["offsets"]) and np.array_equal(srt, f["sorted"]) and np.array_equal(pos, f["pos"])
    ci, cs = c_oracle.route(f["logits"], 8)
    assert np.array_equal(ci, f["inds"])


def test_gather_fixture():
    f = _load("gather_qmm")
    x = quant_ref.bf16_from_bits(f["x"])
    s, b = quant_ref.bf16_from_bits(f["s"]), quant_ref.bf16_from_bits(f["b"])
    rows = np.repeat(np.arange(6), 2)
    y = moe_ref.gather_qmm(x, rows.tolist(), f["inds"].reshape(-1).tolist(), f["w"], s, b, 4)
    assert np.array_equal(quant_ref.bf16_bits(y), f["y"])


def test_verify_trace_fixture():
    f = _load("verify_trace")
    committed = [int(f["greedy"][0])]
    for draft, tt, n in zip(f["drafts"], f["tts"], f["n"]):
        d = [int(t) for t in draft if t >= 0]
        t = [int(v) for v in tt if v >= 0]
        got_n, c = verify_ref.greedy_accept(d, t)
        assert got_n == n
        committed += c
    assert committed == f["committed"].tolist()
    assert committed[:60] == f["greedy"][:60].tolist()           # lossless: the greedy sequence
    rounds = len(f["n"])
    assert verify_ref.mean_accept_len(len(committed) - 1, rounds) == float(f["mean_accept_len"][0])
    assert int(f["offsets_end"][0]) == 5 + len(committed) - 1
