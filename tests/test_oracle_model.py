"""Pins oracle/model_ref.py: RMSNorm and RoPE closed forms and invariants, rollback semantics of
the numpy forward, and agreement of the numpy forward with the torch module path of the same
weights on the CPU (two independent implementations of mlx-lm's decoder semantics)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _model_util import tiny_model, to_ref
from _util import ROPE_KAT_TOL, rope_kat_errors
from oracle import model_ref, quant_ref


def test_rmsnorm_closed_form():
    x = np.full((2, 64), 3.0, dtype=np.float32)
    x[1] = -0.5
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    y = model_ref.rmsnorm(x, quant_ref.bf16_round(w), 1e-6)
    assert np.allclose(y[0], quant_ref.bf16_round(w), rtol=2 ** -7)
    assert np.allclose(y[1], -quant_ref.bf16_round(w), rtol=2 ** -7)
    r = np.random.Generator(np.random.PCG64(0)).standard_normal((3, 128)).astype(np.float32)
    yy = model_ref.rmsnorm(quant_ref.bf16_round(r), np.ones(128, np.float32), 1e-6)
    assert np.allclose(np.sqrt((yy.astype(np.float64) ** 2).mean(-1)), 1.0, atol=1e-2)


def test_rope_invariants():
    r = np.random.Generator(np.random.PCG64(1))
    x = quant_ref.bf16_round(r.standard_normal((2, 5, 128)).astype(np.float32))
    assert np.array_equal(model_ref.rope(x[:, :1], [0], 1e6), x[:, :1])            # position 0: identity
    y = model_ref.rope(x, np.arange(5) + 1000, 1e6)
    n0 = x[..., :64] ** 2 + x[..., 64:] ** 2
    n1 = y[..., :64].astype(np.float64) ** 2 + y[..., 64:].astype(np.float64) ** 2
    assert np.allclose(n1, n0, rtol=2e-2, atol=1e-3)                              # rotations keep pair norms
    q, k = x[0, :1], x[1, :1]
    dots = [float(np.sum(model_ref.rope(q, [p + 7], 1e4).astype(np.float64) *
                         model_ref.rope(k, [p], 1e4).astype(np.float64))) for p in (0, 33, 500)]
    assert max(dots) - min(dots) < 0.05 * np.abs(q).sum()                         # relative position only


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("base", [1e4, 1e6])
def test_rope_frequency_schedule_closed_form(D, base):
    assert rope_kat_errors(model_ref.rope, D, base) <= ROPE_KAT_TOL


def test_rope_kat_rejects_wrong_schedules():
    """The KAT fails a plausible slip: the exponent -i/D instead of -2i/D, or the wrong base."""
    def wrong_exponent(x, pos, base):
        x = np.asarray(x, np.float32)
        D = x.shape[-1]
        half = D // 2
        inv = base ** (-np.arange(half) / D)
        ang = np.asarray(pos, np.float64)[:, None] * inv[None, :]
        c, s = np.cos(ang), np.sin(ang)
        x1, x2 = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
        return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)

    def wrong_base(x, pos, base):
        return model_ref.rope(x, pos, base * 10)

    def traditional_pairs(x, pos, base):   # pairs (2i, 2i+1) instead of (i, i + D/2)
        x = np.asarray(x, np.float64)
        D = x.shape[-1]
        inv = base ** (-2.0 * np.arange(D // 2) / D)
        ang = np.asarray(pos, np.float64)[:, None] * inv[None, :]
        c, s = np.cos(ang), np.sin(ang)
        y = x.copy()
        y[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
        y[..., 1::2] = x[..., 0::2] * s + x[..., 1::2] * c
        return y

    for fn in (wrong_exponent, wrong_base, traditional_pairs):
        assert rope_kat_errors(fn, 128, 1e6) > 10 * ROPE_KAT_TOL, fn.__name__


def test_numpy_forward_matches_torch_module_path_on_cpu():
    model = tiny_model("cpu", seed=3)
    ref = to_ref(model)
    cache = model.make_cache(64)
    ids = [5, 17, 200, 3, 99, 41]
    with torch.no_grad():
        got = model(torch.tensor([ids]), cache)[0].float().numpy()
    want = ref.forward(ids)
    rms = np.sqrt(np.mean(want.astype(np.float64) ** 2))
    assert np.abs(got - want).max() <= 2e-2 * rms
    # a second verify block at offset 6 over the cached rows
    with torch.no_grad():
        got2 = model(torch.tensor([[7, 8, 9]]), cache)[0].float().numpy()
    want2 = ref.forward([7, 8, 9])
    assert np.abs(got2 - want2).max() <= 2e-2 * np.sqrt(np.mean(want2.astype(np.float64) ** 2))


def test_rollback_equals_fresh_prefix():
    model = tiny_model("cpu", seed=4)
    a = to_ref(model)
    a.forward([1, 2, 3, 4, 5])
    a.trim(2)                                    # keep [1, 2, 3]
    la = a.forward([9, 10])
    b = to_ref(model)
    b.forward([1, 2, 3])
    lb = b.forward([9, 10])
    assert np.array_equal(la, lb)


def test_c_matmul_and_seeded_cache_agree_with_the_numpy_forward():
    """qmm_c (the C restatement) lands within one bf16 rounding of the float64 qmm on every
    projection, and a forward whose caches are seeded with a prefix equals the forward that
    wrote that prefix itself (the seeded rows are what the earlier forward cached)."""
    model = tiny_model("cpu", seed=11)
    r = np.random.Generator(np.random.PCG64(2))
    lin = to_ref(model).layers[0]["gate"]
    x = quant_ref.bf16_round(r.standard_normal((5, model.args.hidden_size)).astype(np.float32))
    a, b = model_ref.qmm(x, lin), model_ref.qmm_c(x, lin)
    assert np.all(np.abs(a - b) <= 2 ** -7 * np.abs(a) + 1e-6)
    full = to_ref(model, matmul=model_ref.qmm_c)
    full.forward([4, 8, 15, 16, 23])
    seeded = to_ref(model, matmul=model_ref.qmm_c)
    seeded.seed_cache([k[:, :5] for k in full.k], [v[:, :5] for v in full.v])
    assert seeded.offset == 5
    assert np.array_equal(seeded.forward([42, 7]), full.forward([42, 7]))


def test_quantized_kv_forward_matches_torch_module_path_on_cpu():
    """The oracle's quantized-cache forward (rows quantized with quant_ref's rule, dequantized
    exactly) against the torch module path over QuantizedKVCache on the CPU (quant.quantize_rows,
    then the stock quantized SDPA): two implementations of the same cache semantics. Bar: the
    whole forward's 5e-2 x RMS (a key that rounds to a neighbouring field moves by a whole
    quantization step, which the two-layer forward then carries)."""
    for bits in (8, 4):
        model = tiny_model("cpu", seed=17)
        ref = to_ref(model, kv_bits=bits)
        cache = model.make_cache(64, kv_bits=bits)
        for ids in ([5, 17, 200, 3, 99, 41], [7, 8, 9]):
            with torch.no_grad():
                got = model(torch.tensor([ids]), cache)[0].float().numpy()
            want = ref.forward(ids)
            assert np.abs(got - want).max() <= 5e-2 * np.sqrt(np.mean(want.astype(np.float64) ** 2)), bits
