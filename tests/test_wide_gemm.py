"""CPU tests of the prefill wide path's scope and calibration logic (dspark_rocm.wide_gemm),
mirroring the reference's tests/test_wide_gemm.py:37-200: no-op when disabled, patch / restore
/ exception / nesting, the row floor, leading dims counted as rows, eligibility, the widest
weight, and the crossover invariant (whatever threshold calibration returns verified there).
The kernel-backed cases (bit identity across dtypes and widths, bias, the real crossover) are
in test_gpu_wide_gemm.py."""

from __future__ import annotations

import pytest
import torch

from dspark_rocm import wide_gemm as wg
from dspark_rocm.nn import QuantizedLinear

K, N = 256, 128


def _lin(n=N, k=K, bits=8, bias=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    return QuantizedLinear.random(n, k, bits=bits, generator=g, bias=bias)


def test_disabled_is_a_noop():
    for arg in (None, 0):
        with wg.wide_matmul(arg):
            assert not wg.active()
    assert QuantizedLinear.forward is wg._orig_call


def test_patch_applies_and_restores():
    assert not wg.active()
    with wg.wide_matmul(64):
        assert wg.active()
    assert not wg.active() and QuantizedLinear.forward is wg._orig_call


def test_patch_restores_on_exception():
    with pytest.raises(RuntimeError), wg.wide_matmul(64):
        raise RuntimeError("boom")
    assert not wg.active() and QuantizedLinear.forward is wg._orig_call


def test_nested_scope_does_not_restore_early():
    with wg.wide_matmul(64):
        cfg = wg._cfg.value
        with wg.wide_matmul(1024):            # already active: the inner scope leaves it alone
            assert wg.active() and wg._cfg.value is cfg
        assert wg.active()
    assert not wg.active()


def test_nests_inside_small_m_and_restores_it():
    """A prefill inside a decode loop: the wide scope falls through to, and restores, the
    small-M patch it found (wide_gemm.py:221-223)."""
    from dspark_rocm import small_m_qmm

    with small_m_qmm.small_m_matmul(frozenset({1})):
        below = QuantizedLinear.forward
        with wg.wide_matmul(256):
            assert wg.active() and wg._below.value is below
        assert QuantizedLinear.forward is below
    assert QuantizedLinear.forward is wg._orig_call


def test_floor_is_enforced_against_the_flag():
    with wg.wide_matmul(8):
        assert wg._cfg.value[0] == wg.SAFE_MIN_ROWS
    with wg.wide_matmul(4096, shapes=["a"]):
        assert wg._cfg.value[:2] == (4096, frozenset({"a"}))


def test_routing_decision_counts_leading_dims_and_shapes(monkeypatch):
    lin = _lin()
    monkeypatch.setattr(torch.Tensor, "is_cuda", property(lambda self: True))
    with wg.wide_matmul(256):
        assert wg.serves(lin, torch.empty(1, 256, K))        # [1, L, K]: L rows, not 1
        assert wg.serves(lin, torch.empty(2, 128, K))
        assert not wg.serves(lin, torch.empty(1, 255, K))
    with wg.wide_matmul(256, shapes=[wg.shape_key(lin)]):
        assert wg.serves(lin, torch.empty(256, K))
    with wg.wide_matmul(256, shapes=["1x1x8xbfloat16"]):
        assert not wg.serves(lin, torch.empty(256, K))       # not verified: stock path
    assert not wg.serves(lin, torch.empty(256, K))           # no scope


def test_cpu_and_narrow_inputs_fall_through_unchanged():
    lin = _lin(bias=True)
    for rows in (2, 300):
        x = torch.randn(rows, K).to(torch.bfloat16)
        ref = lin(x)
        with wg.wide_matmul(256):
            got = lin(x)                                      # a CPU tensor never takes the kernel
        assert torch.equal(got, ref)


def test_shape_key_and_eligibility():
    lin = _lin(bits=4)
    assert wg.shape_key(lin) == f"{K}x{N}x4xbfloat16"
    assert wg._eligible(lin)
    lin.mode = "mxfp4"
    assert not wg._eligible(lin)
    nob = _lin()
    nob.biases = None
    assert not wg._eligible(nob)
    assert list(wg.quantized_linears(torch.nn.Sequential(lin, nob))) == []


def test_widest_quantized_linear_picks_the_biggest_and_looks_through_model():
    model = torch.nn.Sequential(_lin(512, K), _lin(2048, K), _lin(256, K))
    assert int(wg.widest_quantized_linear(model).weight.shape[0]) == 2048

    class Holder:
        pass

    h = Holder()
    h.model = model
    assert wg.widest_quantized_linear(h) is wg.widest_quantized_linear(model)
    assert wg.widest_quantized_linear(torch.nn.Sequential(torch.nn.Linear(8, 8))) is None
    assert wg.measure_crossover(torch.nn.Sequential(torch.nn.Linear(8, 8))) is None


def _fake_timing(monkeypatch, wins_from: int):
    """The race on the widest weight: the wide path wins from ``wins_from`` rows."""
    seen = []

    def fake_wins(lin, M, gen, exact, margin):
        seen.append(M)
        return M >= wins_from

    monkeypatch.setattr(wg, "_wide_wins", fake_wins)
    return seen


def test_crossover_never_returns_a_threshold_that_is_not_identical(monkeypatch):
    """The reference's invariant (tests/test_wide_gemm.py:140-165): the only shape differs at
    the floor, so calibration refuses or moves wider to a width where it does verify."""
    model = torch.nn.Sequential(_lin(1024, K))
    _fake_timing(monkeypatch, wins_from=256)
    monkeypatch.setattr(wg, "_agrees", lambda mod, M, exact=True: M != wg.SAFE_MIN_ROWS)
    assert wg.verified_shapes([model], wg.SAFE_MIN_ROWS, widths=()) == []
    got = wg.measure_crossover(model)
    assert got is None or (got[0] > wg.SAFE_MIN_ROWS and wg.verified_shapes([model], got[0], widths=()) == got[1])


def test_crossover_picks_the_first_width_that_keeps_winning(monkeypatch):
    model = torch.nn.Sequential(_lin(1024, K), _lin(512, K, bits=4))
    seen = _fake_timing(monkeypatch, wins_from=1024)
    monkeypatch.setattr(wg, "_agrees", lambda mod, M, exact=True: True)
    got = wg.measure_crossover(model, widths=(128, 256, 512, 1024, 2048))
    assert got == (1024, [f"{K}x1024x8xbfloat16", f"{K}x512x4xbfloat16"])
    assert seen == [256, 512, 1024, 2048]                      # under the floor: never raced
    assert wg.gate.winning_tail([False, True, False, True, True]) == 3
    assert wg.gate.winning_tail([True, True]) == 0 and wg.gate.winning_tail([True, False]) is None
    _fake_timing(monkeypatch, wins_from=10 ** 9)                # never faster: off
    assert wg.measure_crossover(model) is None


def test_verified_shapes_drops_a_shape_whose_kernel_raises(monkeypatch):
    model = torch.nn.Sequential(_lin(1024, K), _lin(512, K))

    def agrees(mod, M, exact=True):
        if int(mod.weight.shape[0]) == 512:
            raise RuntimeError("refused")
        return True

    monkeypatch.setattr(wg, "_agrees", agrees)
    assert wg.verified_shapes([model], 256) == [f"{K}x1024x8xbfloat16"]
