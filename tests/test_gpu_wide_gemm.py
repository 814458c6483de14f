"""GPU: the prefill wide path (dspark_rocm.wide_gemm) and its dequantize kernel.

- ``dspark_qmm_dequantize`` against the oracle's exact (float64) dequantization: for bf16 and
  fp16 scales ``scale * q`` is exact in fp32, so the kernel's fp32 output is the float64 value
  rounded once; for fp32 scales it is numpy's float32 product rounded, then sum rounded; the
  bf16 / fp16 outputs are that fp32 value rounded to the dtype;
- the reference's load-bearing property (tests/test_wide_gemm.py:74-88): inside the scope the
  result is bit-identical to the stock path for fp32 / fp16 / bf16 activations at 4 and 8 bits,
  over [1, L, K] leading dims, with a module bias; narrow calls fall through unchanged;
- the verification accepts a shape where the paths agree and calibration never returns a
  threshold that does not verify (the divergence is simulated at the floor);
- the exact=False variant (bf16 GEMM) within the qmm bar;
- ``Target.prefill`` fills the caches identically with the wide path on and off.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import quant_ref

pytestmark = pytest.mark.gpu

K, N, ROWS = 4096, 4096, 256


def _lin_at(dev, dtype, bits, n=N, k=K, bias=False, seed=0):
    """A QuantizedLinear quantized at ``dtype`` (scales and biases in that dtype), as a
    converted checkpoint of that dtype holds it."""
    from dspark_rocm.nn import QuantizedLinear
    from dspark_rocm.quant import quantize_rows

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = torch.randn((n, k), generator=g, device=dev) * 0.02
    wq, s, b = quantize_rows(w, bits, dtype=dtype)
    bb = (torch.randn(n, generator=g, device=dev) * 0.02).to(dtype) if bias else None
    return QuantizedLinear(wq, s, b, bb, bits=bits)


@pytest.mark.parametrize("sdt", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("bits", [4, 8])
def test_dequantize_kernel_matches_the_oracle(dev, sdt, bits):
    from dspark_rocm import ops, quant

    lin = _lin_at(dev, sdt, bits, n=192, k=1024, seed=bits)
    w = lin.weight.cpu().numpy().view(np.uint32)
    s = lin.scales.float().cpu().numpy()
    b = lin.biases.float().cpu().numpy()
    if sdt == torch.float32:
        q = quant_ref.unpack(w, bits).astype(np.float32).reshape(192, 16, 64)
        want = (q * s[..., None] + b[..., None]).reshape(192, 1024)      # float32: rounded per op
    else:
        want = quant_ref.dequantize(w, s, b, bits).astype(np.float32)    # float64 rounded once
    got = ops.dequantize(lin.weight, lin.scales, lin.biases, bits=bits, dtype=torch.float32)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    assert torch.equal(got, quant.dequantize(lin.weight, lin.scales, lin.biases, bits=bits))
    for dt in (torch.bfloat16, torch.float16):
        half = ops.dequantize(lin.weight, lin.scales, lin.biases, bits=bits, dtype=dt)
        assert torch.equal(half, torch.from_numpy(want).to(dev).to(dt))
    # a strided destination: rows of a wider buffer
    buf = torch.full((192, 1024 + 64), 7.0, device=dev)
    ops.dequantize(lin.weight, lin.scales, lin.biases, bits=bits, dtype=torch.float32, out=buf[:, :1024])
    assert torch.equal(buf[:, :1024], got) and bool((buf[:, 1024:] == 7.0).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits", [4, 8])
def test_bit_identical_above_threshold(dev, bits, dtype):
    from dspark_rocm import wide_gemm as wg

    lin = _lin_at(dev, dtype, bits)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    x = torch.randn((ROWS, K), generator=g, device=dev).to(dtype)
    ref = lin(x)
    calls = []
    real = wg.wide_rows
    with wg.wide_matmul(ROWS), torch.no_grad():
        wg.wide_rows = lambda *a, **k: calls.append(1) or real(*a, **k)
        try:
            got = lin(x)
        finally:
            wg.wide_rows = real
    assert calls, "the forward did not take the wide path"
    assert got.shape == ref.shape and torch.equal(got, ref)


def test_leading_dims_bias_and_narrow_fall_through(dev):
    from dspark_rocm import wide_gemm as wg

    lin = _lin_at(dev, torch.bfloat16, 8, bias=True)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    x3 = torch.randn((1, ROWS, K), generator=g, device=dev).to(torch.bfloat16)
    x_narrow = torch.randn((64, K), generator=g, device=dev).to(torch.bfloat16)
    ref3, refn = lin(x3), lin(x_narrow)
    with wg.wide_matmul(8):                          # clamped to the floor: 64 rows fall through
        assert wg.serves(lin, x3) and not wg.serves(lin, x_narrow)
        got3, gotn = lin(x3), lin(x_narrow)
    assert got3.shape == (1, ROWS, N) and torch.equal(got3, ref3)
    assert torch.equal(gotn, refn)


def test_verified_shapes_and_crossover_invariant(dev, monkeypatch):
    from dspark_rocm import wide_gemm as wg

    model = torch.nn.Sequential(_lin_at(dev, torch.bfloat16, 8), _lin_at(dev, torch.bfloat16, 4, n=1024))
    keys = wg.verified_shapes([model], wg.SAFE_MIN_ROWS, widths=(512,))
    assert keys == [f"{K}x{N}x8xbfloat16", f"{K}x1024x4xbfloat16"]
    got = wg.measure_crossover(model)
    print("measured crossover:", got, flush=True)
    assert got is None or (got[0] >= wg.SAFE_MIN_ROWS and got[1] == keys)
    real = wg._agrees
    monkeypatch.setattr(wg, "_agrees", lambda mod, M, exact=True: M != wg.SAFE_MIN_ROWS and real(mod, M, exact))
    assert wg.verified_shapes([model], wg.SAFE_MIN_ROWS, widths=()) == []
    got = wg.measure_crossover(model)
    assert got is None or (got[0] > wg.SAFE_MIN_ROWS and wg.verified_shapes([model], got[0], widths=()) == got[1])


@pytest.mark.parametrize("bits", [4, 8])
def test_half_gemm_variant_within_the_qmm_bar(dev, bits):
    from dspark_rocm import wide_gemm as wg

    lin = _lin_at(dev, torch.bfloat16, bits, bias=True)
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    x = torch.randn((512, K), generator=g, device=dev).to(torch.bfloat16)
    ref = lin(x).float()
    with wg.wide_matmul(256, exact=False):
        got = lin(x).float()
    d = float((got - ref).abs().max())
    assert 0 < d <= wg.REL_TOL * max(float(ref.abs().max()), 1.0)
    assert wg.verified_shapes([torch.nn.Sequential(lin)], 256, widths=(), exact=False) == [wg.shape_key(lin)]


def test_prefill_fills_caches_identically_with_the_wide_path(dev, monkeypatch):
    """prefill_plain (Target.prefill per chunk) with the wide path forced on (every shape verified at 256 rows) leaves
    bit-identical caches and logits to the stock prefill, over two chunks (300 + 300 rows)."""
    from _model_util import tiny_model

    from dspark_rocm import calibrate, wide_gemm
    from dspark_rocm.model import Target, prefill_plain

    model = tiny_model(dev, seed=21, hidden_size=512, intermediate_size=1536)
    tgt = Target(model)
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, model.args.vocab_size, (1, 600), generator=g)
    monkeypatch.setattr(calibrate, "WIDE_GEMM_MIN_ROWS", None)
    monkeypatch.setattr(calibrate, "WIDE_GEMM_SHAPES", None)
    stock_cache = tgt.make_cache(640)
    with torch.no_grad():
        stock, _ = prefill_plain(tgt, ids, stock_cache, chunk=300)
    assert calibrate.apply_wide_gemm(model, target_repo="synthetic", min_rows=256, verbose=False) == 256
    assert len(calibrate.WIDE_GEMM_SHAPES) == len({wide_gemm.shape_key(m) for m in wide_gemm.quantized_linears(model)})
    n = []
    real = wide_gemm.wide_rows
    monkeypatch.setattr(wide_gemm, "wide_rows", lambda *a, **k: n.append(1) or real(*a, **k))
    wide_cache = tgt.make_cache(640)
    with torch.no_grad():
        wide, _ = prefill_plain(tgt, ids, wide_cache, chunk=300)
    assert n, "no projection took the wide path"
    assert stock.shape == (1, 1, model.args.vocab_size) and torch.equal(wide, stock)
    for a, b in zip(stock_cache, wide_cache):
        assert a.offset == b.offset == 600
        ka, va = a.fetch()
        kb, vb = b.fetch()
        assert torch.equal(ka, kb) and torch.equal(va, vb)
