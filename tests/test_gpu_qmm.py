"""GPU parity of the small-M affine qmm (dspark_qmm_affine / _multi) against the oracle.

Bar: max|Δ| <= 2e-2 * RMS(y) (bf16 out, fp32 accumulate); in practice the kernel lands within
a couple of bf16 ulps, which the tighter per-element check below pins. Structure mirrors the
reference's tests/test_small_m_qmm.py: every M of the window at both widths (:59-87), bitwise
row-count invariance (:107-119), ragged N, the refusal paths, plus the full-size 4096 x 4096 shape.
"""

from __future__ import annotations

import numpy as np
import pytest

from _util import assert_rms_close, from_dev_bf16, randn_bf16, rng, to_dev_bf16, to_dev_packed
from oracle import c_oracle, qmm_ref, quant_ref

pytestmark = pytest.mark.gpu


def _problem(seed, m, k, n, bits, quantized=False):
    r = rng(seed)
    x = randn_bf16(r, m, k)
    if quantized:
        w32 = (r.standard_normal((n, k)) * 0.02).astype(np.float32)
        w, s, b = quant_ref.quantize(w32, bits)
    else:
        w, s, b = quant_ref.random_packed(r, n, k, bits)
    return x, w, s, b


def _run(dev, x, w, s, b, bits):
    from dspark_rocm import ops

    y = ops.quantized_matmul(to_dev_bf16(x, dev), to_dev_packed(w, dev), to_dev_bf16(s, dev),
                             to_dev_bf16(b, dev), bits=bits)
    return from_dev_bf16(y)


def _check(got, ref_f64, what):
    ref = quant_ref.bf16_round(ref_f64.astype(np.float32))
    assert_rms_close(got, ref, 2e-2, what)
    # tight: within 2 bf16 ulps of the exact result (+ a floor for values near zero)
    tol = 2.0 ** -7 * np.abs(ref_f64) + 1e-3 * qmm_ref.rms(ref_f64)
    bad = np.abs(got - ref_f64) > tol
    assert not bad.any(), f"{what}: {bad.sum()} elements beyond 2 ulps, worst {np.max(np.abs(got - ref_f64)):.4g}"


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 15, 16])
def test_window_numerics(dev, bits, m):
    x, w, s, b = _problem(100 + m, m, 512, 4096, bits, quantized=True)
    got = _run(dev, x, w, s, b, bits)
    _check(got, qmm_ref.qmm_f64(x, w, s, b, bits), f"{bits}-bit M={m}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("k,n", [(64, 8), (192, 72), (256, 64), (768, 2048), (2048, 768), (12288, 128),
                                 (32768, 96)])   # the largest K: 32 slices of 16 groups
def test_shapes(dev, bits, k, n):
    x, w, s, b = _problem(7 * k + n, 16, k, n, bits)
    got = _run(dev, x, w, s, b, bits)
    _check(got, qmm_ref.qmm_f64(x, w, s, b, bits), f"{bits}-bit {k}x{n}")


@pytest.mark.parametrize("bits", [4, 8])
def test_rows_are_row_count_invariant(dev, bits):
    """A row's result does not depend on how many rows ride with it (bitwise)."""
    x, w, s, b = _problem(5, 16, 1024, 512, bits)
    full = _run(dev, x, w, s, b, bits)
    for m in range(1, 16):
        part = _run(dev, x[:m], w, s, b, bits)
        assert np.array_equal(full[:m], part), (bits, m)


@pytest.mark.parametrize("bits", [4, 8])
def test_more_than_16_rows(dev, bits):
    x, w, s, b = _problem(11, 37, 512, 256, bits)
    got = _run(dev, x, w, s, b, bits)
    _check(got, qmm_ref.qmm_f64(x, w, s, b, bits), "M=37")
    assert np.array_equal(got[:16], _run(dev, x[:16], w, s, b, bits))


@pytest.mark.parametrize("bits", [4, 8])
def test_4096x4096_full_size_against_c_oracle(dev, bits):
    """M=16, N=K=4096 (the C restatement, fp32 factored like the kernel)."""
    x, w, s, b = _problem(0, 16, 4096, 4096, bits)
    got = _run(dev, x, w, s, b, bits)
    ref = c_oracle.qmm(quant_ref.bf16_bits(x), w, quant_ref.bf16_bits(s), quant_ref.bf16_bits(b), bits)
    _check(got, ref.astype(np.float64), f"4096x4096 {bits}-bit")


@pytest.mark.parametrize("bits", [4, 8])
def test_multi_matches_separate_calls(dev, bits):
    import torch

    from dspark_rocm import ops

    r = rng(3)
    x = to_dev_bf16(randn_bf16(r, 16, 1024), dev)
    mats = [quant_ref.random_packed(r, n, 1024, bits) for n in (512, 128, 128)]
    ws = [to_dev_packed(w, dev) for w, _, _ in mats]
    ss = [to_dev_bf16(s, dev) for _, s, _ in mats]
    bs = [to_dev_bf16(b, dev) for _, _, b in mats]
    multi = ops.quantized_matmul_multi([x], ws, ss, bs, bits=bits)
    for i in range(3):
        single = ops.quantized_matmul(x, ws[i], ss[i], bs[i], bits=bits)
        assert torch.equal(multi[i], single), i


C2_SHAPES = [(4096, 4096), (1024, 4096), (12288, 4096), (4096, 12288)]   # [N, K] of the 8B-shaped layer set


@pytest.mark.parametrize("m", [1, 4, 8, 16])
@pytest.mark.parametrize("n,k", C2_SHAPES)
def test_8b_layer_set_shapes_against_c_oracle(dev, n, k, m):
    """Every distinct [N, K] of the 8-bit layer set (q/o, k/v, gate/up, down) at each verify
    width, against the C restatement: the whole-K launch ([4096, 4096]) and the split-K plans."""
    x, w, s, b = _problem(n + k + m, m, k, n, 8, quantized=True)
    got = _run(dev, x, w, s, b, 8)
    ref = c_oracle.qmm(quant_ref.bf16_bits(x), w, quant_ref.bf16_bits(s), quant_ref.bf16_bits(b), 8)
    _check(got, ref.astype(np.float64), f"8-bit {n}x{k} M={m}")


def test_multi_with_outlier_x_within_tolerance(dev):
    """x whose groups of 64 span many binades (values near 1e3 and 1e-3 in one group): an 8-bit
    [4096, 4096] matrix launched alone (whole-K) and inside a q/k/v launch (split-K) may differ
    by an fp32 rounding of the bias term; both stay within 2 ulps of the exact result."""
    from dspark_rocm import ops

    r = rng(17)
    x = randn_bf16(r, 16, 4096)
    x[:, ::64] *= 1e3
    x[:, 1::64] *= 1e-3
    x = quant_ref.bf16_round(x)
    mats = [quant_ref.random_packed(r, n, 4096, 8) for n in (4096, 1024, 1024)]
    xd = to_dev_bf16(x, dev)
    wd = [to_dev_packed(w, dev) for w, _, _ in mats]
    sd = [to_dev_bf16(s, dev) for _, s, _ in mats]
    bd = [to_dev_bf16(b, dev) for _, _, b in mats]
    multi = ops.quantized_matmul_multi([xd], wd, sd, bd, bits=8)
    for i, (w, s, b) in enumerate(mats):
        single = ops.quantized_matmul(xd, wd[i], sd[i], bd[i], bits=8)
        ref = qmm_ref.qmm_f64(x, w, s, b, 8)
        _check(from_dev_bf16(single), ref, f"alone {i}")
        _check(from_dev_bf16(multi[i]), ref, f"in the multi launch {i}")


def test_strided_x_rows(dev):
    """x with a row stride larger than K (a view into a wider buffer)."""
    import torch

    from dspark_rocm import ops

    x, w, s, b = _problem(9, 8, 512, 128, 4)
    xb = to_dev_bf16(np.concatenate([x, np.zeros((8, 64), np.float32)], axis=1), dev)[:, :512]
    y = ops.quantized_matmul(xb, to_dev_packed(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev), bits=4)
    assert torch.equal(y, ops.quantized_matmul(xb.contiguous(), to_dev_packed(w, dev), to_dev_bf16(s, dev),
                                               to_dev_bf16(b, dev), bits=4))


def test_refusals_raise(dev):
    import torch

    from dspark_rocm import _lib, ops

    x = torch.zeros((4, 96), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((8, 12), dtype=torch.int32, device=dev)
    s = torch.zeros((8, 1), dtype=torch.bfloat16, device=dev)
    with pytest.raises((_lib.DsparkError, ValueError)):
        ops.quantized_matmul(x, w, s, s, bits=4)          # K = 96 is not a multiple of 64
    lib = _lib.load()
    assert lib.dspark_qmm_affine_supported(4, 128, 8, 2, 64) == -6
    assert lib.dspark_qmm_affine_supported(4, 96, 8, 4, 64) == -2
    assert lib.dspark_qmm_affine_supported(4, 128, 8, 4, 32) == -6
    assert lib.dspark_qmm_affine_supported(16, 4096, 4096, 8, 64) == 0


@pytest.mark.parametrize("bits", [4, 8])
def test_split_k_workspace_reuse_is_bitwise_stable(dev, bits):
    """Shapes that split K across workgroups share one workspace; its arrival counters must be
    left at zero by every call, so repeated and interleaved calls give identical bits (the 8-bit
    [4096, 4096] launch, which splits nothing, is interleaved with them). The
    8192-row shape has 128 strip counters, more than the others: their partials must not land
    on its counters."""
    import torch

    from dspark_rocm import _lib, ops

    shapes = [(4096, 4096), (8192, 1024), (1024, 4096), (4096, 12288), (256, 2048)]
    inputs = []
    for i, (n, k) in enumerate(shapes):
        x, w, s, b = _problem(50 + i, 16, k, n, bits)
        # (the [4096, 4096] launch takes no workspace: one whole-K workgroup per 16-row tile)
        whole_k = (n, k) == (4096, 4096)
        assert (_lib.load().dspark_qmm_affine_workspace(16, k, n, bits, 64) > 0) != whole_k or n * k < 2**20
        inputs.append(tuple(t(v, dev) for t, v in zip((to_dev_bf16, to_dev_packed, to_dev_bf16, to_dev_bf16),
                                                         (x, w, s, b))) + ((x, w, s, b),))
    first = [ops.quantized_matmul(xd, wd, sd, bd, bits=bits) for xd, wd, sd, bd, _ in inputs]
    for rep in range(3):
        for i in ([0, 1, 2, 3, 4] if rep % 2 == 0 else [3, 1, 4, 0, 2]):
            xd, wd, sd, bd, _ = inputs[i]
            again = ops.quantized_matmul(xd, wd, sd, bd, bits=bits)
            assert torch.equal(again, first[i]), (rep, i)
    for (xd, wd, sd, bd, host), y in zip(inputs, first):
        _check(from_dev_bf16(y), qmm_ref.qmm_f64(*host, bits), "split-K")


def test_workspace_reset_restores_counters(dev):
    """dspark_qmm_workspace_reset zeroes the arrival counters of a workspace whose counters hold
    arbitrary values (e.g. after a call that did not complete); the next call is then bitwise the
    call on a fresh zeroed workspace. Only the reset path runs: no launch sees the stale counters."""
    import torch

    from dspark_rocm import ops

    from dspark_rocm import _lib

    # a split-K shape (8-bit 6144 x 4096: K slices, arrival counters and partials in the workspace)
    assert _lib.load().dspark_qmm_affine_workspace(16, 4096, 6144, 8, 64) > 0
    x, w, s, b = _problem(61, 16, 6144, 4096, 8)
    xd, wd, sd, bd = to_dev_bf16(x, dev), to_dev_packed(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev)
    want = ops.quantized_matmul(xd, wd, sd, bd, bits=8)
    ws = ops.new_qmm_workspace(dev, 8 << 20)
    ws[: 256 << 10].fill_(7)                       # stale counters
    ops.qmm_workspace_reset(ws)
    torch.cuda.synchronize()
    assert not ws[: 256 << 10].any()
    y = torch.empty_like(want)
    ops.quantized_matmul_multi([xd], [wd], [sd], [bd], bits=8, outs=[y], workspace=ws)
    assert torch.equal(y, want)
    assert not ws[: 256 << 10].any()               # and the call leaves them at zero


def test_stream_read_probe(dev):
    """The bandwidth probe reads without writing its sink (the fold never equals the sentinel
    on these bytes) and refuses sizes that are not whole 16-byte chunks."""
    import torch

    from dspark_rocm import _lib, ops

    buf = torch.arange(1 << 20, dtype=torch.int32, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    ops.stream_read(buf, sink)
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    with pytest.raises(_lib.DsparkError):
        _lib.call("dspark_stream_read", buf.data_ptr(), 20, sink.data_ptr(), 0)
