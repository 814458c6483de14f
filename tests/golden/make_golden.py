"""Writes the committed golden fixtures (tests/golden/*.npz) from seeded numpy inputs and the
oracle restatements (oracle/, pinned by tests/test_oracle_*.py). Run from the repository root:

    python tests/golden/make_golden.py

Fixtures (sizes chosen so the whole set stays small):
  unpack.npz       pack/unpack KATs and a random round trip at 4 and 8 bits
  qmm.npz          affine qmm, M in {1, 5, 8, 16} x (K 256, N 64) x bits {4, 8} (float64 results)
  attention.npz    GQA 8/2 x 128, 16 rows, L in {48, 300}, causal and tree masks (float64)
  route.npz        softmax top-8 of 16 x 128 logits with deliberate ties; bucketing
  gather_qmm.npz   grouped qmm over E = 8 experts, top-2 pairs (bf16-valued fp32)
  verify_trace.npz greedy accept / rollback trace of a 2-layer model (tokens, accepted counts)
The reference (Python + Metal over MLX) cannot run here, so every expected output comes from
the oracle; inputs are drawn with numpy PCG64 so they are identical on every machine.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import attn_ref, moe_ref, qmm_ref, quant_ref, verify_ref  # noqa: E402


def rng(seed):
    return np.random.Generator(np.random.PCG64(seed))


def unpack_fixture():
    r = rng(1)
    out = {"kat4_word": np.array([0x76543210], np.uint32), "kat4_vals": np.arange(8, dtype=np.int32),
           "kat8_word": np.array([0x04030201], np.uint32), "kat8_vals": np.array([1, 2, 3, 4], np.int32)}
    for bits in (4, 8):
        q = r.integers(0, 1 << bits, (8, 64)).astype(np.int32)
        out[f"q{bits}"] = q
        out[f"w{bits}"] = quant_ref.pack(q, bits)
    return out


def qmm_fixture():
    r = rng(2)
    out = {}
    for bits in (4, 8):
        w, s, b = quant_ref.random_packed(r, 64, 256, bits)
        out[f"w{bits}"], out[f"s{bits}"], out[f"b{bits}"] = w, quant_ref.bf16_bits(s), quant_ref.bf16_bits(b)
        for m in (1, 5, 8, 16):
            x = quant_ref.bf16_round(r.standard_normal((m, 256)).astype(np.float32))
            out[f"x{bits}_{m}"] = quant_ref.bf16_bits(x)
            out[f"y{bits}_{m}"] = qmm_ref.qmm_f64(x, w, s, b, bits)
    return out


def attention_fixture():
    r = rng(3)
    out = {}
    anc = np.array([(1 << (i + 1)) - 1 if i % 3 else (1 << i) | 1 for i in range(16)], np.uint32)
    out["tree_anc"] = anc
    for L in (48, 300):
        q = quant_ref.bf16_round(r.standard_normal((1, 8, 16, 128)).astype(np.float32))
        k = quant_ref.bf16_round(r.standard_normal((1, 2, L, 128)).astype(np.float32))
        v = quant_ref.bf16_round(r.standard_normal((1, 2, L, 128)).astype(np.float32))
        out[f"q{L}"], out[f"k{L}"], out[f"v{L}"] = (quant_ref.bf16_bits(t) for t in (q, k, v))
        out[f"causal{L}"] = attn_ref.attention(q, k, v, 128 ** -0.5, causal=True)
        out[f"tree{L}"] = attn_ref.attention(q, k, v, 128 ** -0.5, causal=False, tree_anc=anc)
    return out


def route_fixture():
    r = rng(4)
    x = quant_ref.bf16_round(r.standard_normal((16, 128)).astype(np.float32))
    x[2, [7, 90, 100]] = 4.0            # a three-way tie at the top
    x[5, :] = 0.5                       # every expert tied
    x[9, [3, 4]] = -np.inf              # excluded experts
    inds, scores = moe_ref.route(x, 8)
    off, srt, pos = moe_ref.bucket(inds, 128)
    return {"logits": quant_ref.bf16_bits(x), "inds": inds, "scores": quant_ref.bf16_bits(scores),
            "offsets": off, "sorted": srt, "pos": pos}


def gather_fixture():
    r = rng(5)
    E, N, K = 8, 64, 128
    mats = [quant_ref.random_packed(r, N, K, 4) for _ in range(E)]
    w, s, b = (np.stack([m[i] for m in mats]) for i in range(3))
    x = quant_ref.bf16_round(r.standard_normal((6, K)).astype(np.float32))
    logits = quant_ref.bf16_round(r.standard_normal((6, E)).astype(np.float32))
    inds, _ = moe_ref.route(logits, 2)
    rows = np.repeat(np.arange(6), 2)
    y = moe_ref.gather_qmm(x, rows.tolist(), inds.reshape(-1).tolist(), w, s, b, 4)
    return {"x": quant_ref.bf16_bits(x), "w": w, "s": quant_ref.bf16_bits(s), "b": quant_ref.bf16_bits(b),
            "inds": inds, "y": quant_ref.bf16_bits(y)}


def trace_fixture():
    """Greedy accept/rollback bookkeeping over a fixed token trace (generate.py:1544-1593)."""
    r = rng(6)
    greedy = r.integers(0, 50, 80).tolist()
    pos, rounds, drafts, tts, ns = 0, 0, [], [], []
    committed = [greedy[0]]
    cache = verify_ref.KVCacheRef(1, 128, 2)
    cache.update_and_fetch(np.zeros((1, 5, 2)), np.zeros((1, 5, 2)))     # the prompt
    while len(committed) < 60:
        cap = int(r.integers(1, 8))
        truth = greedy[len(committed):len(committed) + cap]
        draft = [t if r.random() > 0.3 else (t + 1) % 50 for t in truth]
        tt = truth + [greedy[len(committed) + len(truth)]]
        cache.update_and_fetch(np.zeros((1, 1 + len(draft), 2)), np.zeros((1, 1 + len(draft), 2)))
        n, c = verify_ref.greedy_accept(draft, tt)
        verify_ref.rollback([cache], len(draft) - n)
        committed += c
        drafts.append(draft + [-1] * (8 - len(draft)))
        tts.append(tt + [-1] * (9 - len(tt)))
        ns.append(n)
        rounds += 1
    return {"greedy": np.array(greedy), "drafts": np.array(drafts), "tts": np.array(tts), "n": np.array(ns),
            "committed": np.array(committed), "offsets_end": np.array([cache.offset]),
            "mean_accept_len": np.array([verify_ref.mean_accept_len(len(committed) - 1, rounds)])}


def main():
    for name, fn in (("unpack", unpack_fixture), ("qmm", qmm_fixture), ("attention", attention_fixture),
                     ("route", route_fixture), ("gather_qmm", gather_fixture), ("verify_trace", trace_fixture)):
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
