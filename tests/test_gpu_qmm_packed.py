"""GPU: the MI355X packed qmm form (dspark_qmm_pack / dspark_qmm_packed_multi).

- The packed bytes equal a numpy restatement of the layout definition (include/dspark.h,
  csrc/dspark_qmm.hip `pack_kernel`): 16-row weight tiles in MFMA lane order, then 16-row x
  8-group scale/bias tiles, rows past N zero.
- Every product equals the reference-layout kernel's bit for bit (same slices, same per-group
  arithmetic and order), over 4/8 bits, N not a multiple of 16, M = 1..33, multi-problem
  launches; and both are held to the oracle at the qmm bar.
"""

from __future__ import annotations

import functools

import numpy as np
import pytest

from _util import assert_rms_close, from_dev_bf16, randn_bf16, rng, to_dev_bf16, to_dev_packed
from oracle import qmm_ref, quant_ref

pytestmark = pytest.mark.gpu


@functools.lru_cache(maxsize=8)
def _quantized(seed, n, k, bits):
    r = rng(seed)
    w = randn_bf16(r, n, k)
    return quant_ref.quantize(w, bits=bits)          # (packed uint32 [n, k*bits/32], scales, biases)


def _pack_np(wq: np.ndarray, s: np.ndarray, b: np.ndarray, n: int, k: int, bits: int) -> np.ndarray:
    """The packed layout from its definition, with plain numpy indexing."""
    g = k // 64
    t = (n + 15) // 16
    wb = np.ascontiguousarray(wq).view(np.uint8).reshape(n, k * bits // 8)
    sb = np.asarray(quant_ref.bf16_bits(s), dtype=np.uint16).reshape(n, g)
    bb = np.asarray(quant_ref.bf16_bits(b), dtype=np.uint16).reshape(n, g)
    rows = np.zeros((t * 16, wb.shape[1]), dtype=np.uint8)
    rows[:n] = wb
    srows = np.zeros((t * 16, g), dtype=np.uint16)
    brows = np.zeros((t * 16, g), dtype=np.uint16)
    srows[:n], brows[:n] = sb, bb
    out = []
    per_tile = g // 2 if bits == 4 else g
    for ti in range(t):
        for j in range(per_tile):
            for lane in range(64):
                r, q = 16 * ti + (lane & 15), lane >> 4
                if bits == 8:
                    out.append(rows[r, 64 * j + 16 * q: 64 * j + 16 * q + 16])
                else:
                    qs = 2 * (q & 1) + (q >> 1)
                    out.append(np.concatenate([rows[r, 32 * (2 * j) + 8 * qs: 32 * (2 * j) + 8 * qs + 8],
                                               rows[r, 32 * (2 * j + 1) + 8 * qs: 32 * (2 * j + 1) + 8 * qs + 8]]))
    for ti in range(t):
        for o in range(g // 8):
            for arr in (srows, brows):
                for r16 in range(16):
                    out.append(arr[16 * ti + r16, 8 * o: 8 * o + 8].view(np.uint8))
    return np.concatenate(out)


def _dev(wq, s, b, dev):
    return to_dev_packed(wq, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev)


@pytest.mark.parametrize("n,k,bits", [(40, 512, 8), (40, 1024, 4), (16, 512, 4)])
def test_layout_matches_definition(dev, n, k, bits):
    from dspark_rocm import ops

    wq, s, b = _quantized(n + k + bits, n, k, bits)
    pq = ops.qmm_pack(*_dev(wq, s, b, dev), bits=bits)
    got = pq.buf.cpu().numpy()
    want = _pack_np(wq, s, b, n, k, bits)
    assert got.shape == want.shape
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("n,k", [(1000, 512), (4096, 4096), (520, 5120), (64, 25600)])
@pytest.mark.parametrize("m", [1, 5, 16, 33])
def test_bit_identical_to_reference_layout(dev, bits, n, k, m):
    import torch

    from dspark_rocm import ops

    wq, s, b = _quantized(7 * n + k + bits, n, k, bits)
    wd, sd, bd = _dev(wq, s, b, dev)
    x = randn_bf16(rng(m + n), m, k)
    xd = to_dev_bf16(x, dev)
    ref_layout = ops.quantized_matmul(xd, wd, sd, bd, bits=bits)
    packed = ops.quantized_matmul_packed(xd, ops.qmm_pack(wd, sd, bd, bits=bits))
    assert torch.equal(packed, ref_layout)
    if n * k <= 4096 * 4096 and m <= 16:
        want = qmm_ref.qmm_f64(x, wq, s, b, bits)
        assert_rms_close(from_dev_bf16(packed), want, 2e-2, f"packed {bits}-bit [{n},{k}] M={m}")


def test_multi_equals_single(dev):
    import torch

    from dspark_rocm import ops

    k, bits = 4096, 8
    mats = [_dev(*_quantized(i, n, k, bits), dev) for i, n in enumerate((4096, 1024, 1024))]
    packs = [ops.qmm_pack(*m, bits=bits) for m in mats]
    x = to_dev_bf16(randn_bf16(rng(3), 16, k), dev)
    multi = ops.quantized_matmul_packed_multi([x], packs)
    for pq, (wd, sd, bd), y in zip(packs, mats, multi):
        assert torch.equal(y, ops.quantized_matmul_packed(x, pq))
        assert torch.equal(y, ops.quantized_matmul(x, wd, sd, bd, bits=bits))


# K = 4096 launches of 3..6 row tiles per CU take the one-workgroup-per-CU kernel: 768, 1024,
# 1216 (the last workgroup one tile) and 1531 tiles (two problems, the first ending in a half
# tile inside a workgroup that holds the second's first tiles). Its bits are the split-K
# kernel's for the same launch (the reference-layout multi launch: the slice count depends on
# every problem's strips) at every M, and rows of both ends of N are held to the oracle.
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("ns", [(12288,), (16384,), (19456,), (12200, 12288)])
def test_per_cu_kernel_bit_identical_to_split_k(dev, bits, ns):
    import torch

    from dspark_rocm import ops

    k = 4096
    mats = [_quantized(11 * i + bits, n, k, bits) for i, n in enumerate(ns)]
    devs = [_dev(*m, dev) for m in mats]
    packs = [ops.qmm_pack(*d, bits=bits) for d in devs]
    for m in (1, 16, 33):
        x = randn_bf16(rng(m + sum(ns)), m, k)
        wide = torch.zeros((m, k + 64), dtype=torch.bfloat16, device=dev)
        wide[:, 32:32 + k] = to_dev_bf16(x, dev)
        for xd in (to_dev_bf16(x, dev), wide[:, 32:32 + k]):   # contiguous rows, then ldx = K + 64
            plan = ops.packed_multi_plan([xd], packs)
            tiles = sum((n + 15) // 16 for n in ns)
            assert plan["kernel"] == "per CU" and plan["k_parts"] == 1, plan
            assert plan["tiles_per_workgroup"] == -(-tiles // 256)
            got = ops.quantized_matmul_packed_multi([xd], packs)
            want = ops.quantized_matmul_multi([xd], [d[0] for d in devs], [d[1] for d in devs],
                                              [d[2] for d in devs], bits=bits)
            for y, w in zip(got, want):
                assert torch.equal(y, w), (ns, m)
        if m == 16:
            for (wq, s, b), y in zip(mats, got):
                yh = from_dev_bf16(y)
                for sl in (slice(0, 128), slice(wq.shape[0] - 136, wq.shape[0])):
                    want = qmm_ref.qmm_f64(x, wq[sl], s[sl], b[sl], bits)
                    assert_rms_close(yh[:, sl], want, 2e-2, f"per-CU {bits}-bit {ns} rows {sl}")


@pytest.mark.parametrize("bits", [4, 8])
def test_per_cu_kernel_k_parts_bit_identical_to_split_k(dev, bits):
    """The down launch of an 8B-shaped layer ([4096, 12288]: 256 row tiles, 12 slices of 16
    groups) runs four workgroups per group of 4 tiles, each over a quarter of K, the last to
    arrive summing the 12 slices in order: the split-K launch's bits at every M (a second call
    checks the arrival counters were left at zero), rows of both ends of N near the oracle."""
    import torch

    from dspark_rocm import ops

    n, k = 4096, 12288
    wq, s, b = _quantized(91 + bits, n, k, bits)
    d = _dev(wq, s, b, dev)
    pk = ops.qmm_pack(*d, bits=bits)
    for m in (1, 16, 33):
        x = randn_bf16(rng(m + 5), m, k)
        xd = to_dev_bf16(x, dev)
        plan = ops.packed_multi_plan([xd], [pk])
        assert plan["kernel"] == "per CU" and plan["k_parts"] == 4 and plan["tiles_per_workgroup"] == 4, plan
        assert plan["slices"] == 12 and plan["workgroups"] == 256 * ((m + 15) // 16), plan
        want = ops.quantized_matmul_multi([xd], [d[0]], [d[1]], [d[2]], bits=bits)[0]
        for _ in range(2):
            got = ops.quantized_matmul_packed_multi([xd], [pk])[0]
            assert torch.equal(got, want), (bits, m)
        if m == 16:
            yh = from_dev_bf16(got)
            for sl in (slice(0, 64), slice(n - 64, n)):
                ref = qmm_ref.qmm_f64(x, wq[sl], s[sl], b[sl], bits)
                assert_rms_close(yh[:, sl], ref, 2e-2, f"per-CU K parts {bits}-bit rows {sl}")


@pytest.mark.parametrize("m", [1, 16, 33])
def test_per_cu_kernel_two_tiles_8bit(dev, m):
    """The q/k/v launch of an 8B-shaped layer (384 tiles: two per workgroup, K in four parts)
    takes the per-CU kernel at 8 bits only; its bits are the split-K launch's."""
    import torch

    from dspark_rocm import ops

    k, ns = 4096, (4096, 1024, 1024)
    x = to_dev_bf16(randn_bf16(rng(m + 77), m, k), dev)
    for bits, kernel in ((8, "per CU"), (4, "split-K")):
        devs = [_dev(*_quantized(60 + i + bits, n, k, bits), dev) for i, n in enumerate(ns)]
        packs = [ops.qmm_pack(*d, bits=bits) for d in devs]
        plan = ops.packed_multi_plan([x], packs)
        assert plan["kernel"] == kernel, plan
        got = ops.quantized_matmul_packed_multi([x], packs)
        want = ops.quantized_matmul_multi([x], [d[0] for d in devs], [d[1] for d in devs], [d[2] for d in devs],
                                          bits=bits)
        for y, w in zip(got, want):
            assert torch.equal(y, w), (bits, m)


def test_per_cu_kernel_needs_one_x(dev):
    """Problems reading different x tensors, or a launch of too few tiles, keep the split-K
    kernel."""
    from dspark_rocm import ops

    k, bits = 4096, 8
    packs = [ops.qmm_pack(*_dev(*_quantized(40 + i, 12288, k, bits), dev), bits=bits) for i in range(2)]
    x = to_dev_bf16(randn_bf16(rng(5), 16, k), dev)
    assert ops.packed_multi_plan([x], packs)["kernel"] == "per CU"
    assert ops.packed_multi_plan([x, x.clone()], packs)["kernel"] == "split-K"
    small = ops.qmm_pack(*_dev(*_quantized(3, 1024, k, bits), dev), bits=bits)
    assert ops.packed_multi_plan([x], [small])["kernel"] == "split-K"


def test_refusals(dev):
    import torch

    from dspark_rocm import _lib, ops

    assert not ops.qmm_packable(64, 448, 8)          # K % 512 != 0
    assert ops.qmm_packable(64, 512, 4)
    w = torch.zeros((64, 448 // 4), dtype=torch.int32, device=dev)
    s = torch.zeros((64, 7), dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.DsparkError):
        ops.qmm_pack(w, s, s, bits=8)


# ---------------------------------------------------------------- fused gate / up / SwiGLU

def _pair_np(gate, up, n, k, bits):
    """The pair form from its definition: the packed layout of 2 ceil(n/16) tiles, gate tile t
    then up tile t (weights section, then scale/bias section)."""
    a, b = _pack_np(*gate, n, k, bits), _pack_np(*up, n, k, bits)
    t, g = (n + 15) // 16, k // 64
    wt = (g // 2 if bits == 4 else g) * 64 * 16     # weight bytes per tile
    st = (g // 8) * 512                             # scale/bias bytes per tile
    wa, wb = a[:t * wt].reshape(t, wt), b[:t * wt].reshape(t, wt)
    sa, sb = a[t * wt:].reshape(t, st), b[t * wt:].reshape(t, st)
    return np.concatenate([np.stack([wa, wb], 1).reshape(-1), np.stack([sa, sb], 1).reshape(-1)])


@pytest.mark.parametrize("n,k,bits", [(40, 512, 8), (64, 1024, 4)])
def test_swiglu_pair_layout(dev, n, k, bits):
    from dspark_rocm import ops

    gate, up = _quantized(n + 1, n, k, bits), _quantized(n + 2, n, k, bits)
    pair = ops.qmm_pack_swiglu(_dev(*gate, dev), _dev(*up, dev), bits=bits)
    assert np.array_equal(pair.buf.cpu().numpy(), _pair_np(gate, up, n, k, bits))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("n,k", [(1024, 512), (4096, 4096), (640, 5120), (192, 25600)])
@pytest.mark.parametrize("m", [1, 5, 16, 33])
def test_swiglu_fused_is_bitwise_unfused(dev, bits, n, k, m):
    """N a multiple of 64: the fused launch uses the same K slices as the two-problem launch, so
    h equals SwiGLU(gate, up) of the unfused path bit for bit."""
    import torch

    from dspark_rocm import ops

    gate, up = _quantized(3 * n + k + bits, n, k, bits), _quantized(5 * n + k + bits, n, k, bits)
    gd, ud = _dev(*gate, dev), _dev(*up, dev)
    x = randn_bf16(rng(m + 7 * n), m, k)
    xd = to_dev_bf16(x, dev)
    g, u = ops.quantized_matmul_packed_multi([xd], [ops.qmm_pack(*gd, bits=bits), ops.qmm_pack(*ud, bits=bits)])
    want = ops.swiglu(g, u)
    got = ops.quantized_swiglu_packed(xd, ops.qmm_pack_swiglu(gd, ud, bits=bits))
    assert torch.equal(got, want)


@pytest.mark.parametrize("n,k,bits", [(40, 512, 8), (1000, 1024, 4), (24, 2048, 8)])
def test_swiglu_fused_ragged_n_against_oracle(dev, n, k, bits):
    """N not a multiple of 16 (padded tiles; other K slices than the unfused launch): h against
    the oracle's SwiGLU of the oracle products, at the qmm bar."""
    from oracle import moe_ref

    from dspark_rocm import ops

    gate, up = _quantized(n + 11, n, k, bits), _quantized(n + 12, n, k, bits)
    x = randn_bf16(rng(n), 16, k)
    h = ops.quantized_swiglu_packed(to_dev_bf16(x, dev), ops.qmm_pack_swiglu(_dev(*gate, dev), _dev(*up, dev),
                                                                               bits=bits))
    want = moe_ref.swiglu(qmm_ref.qmm_f64(x, *gate, bits), qmm_ref.qmm_f64(x, *up, bits))
    assert_rms_close(from_dev_bf16(h), want, 2e-2, f"fused swiglu {bits}-bit [{n},{k}]")


def test_swiglu_refusals(dev):
    import torch

    from dspark_rocm import _lib, ops

    w = torch.zeros((64, 448 // 4), dtype=torch.int32, device=dev)
    s = torch.zeros((64, 7), dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.DsparkError):                 # K % 512 != 0
        ops.qmm_pack_swiglu((w, s, s), (w, s, s), bits=8)
    w2 = torch.zeros((32, 512 // 4), dtype=torch.int32, device=dev)
    s2 = torch.zeros((32, 8), dtype=torch.bfloat16, device=dev)
    w3 = torch.zeros((64, 512 // 4), dtype=torch.int32, device=dev)
    s3 = torch.zeros((64, 8), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):                       # gate and up shapes differ
        ops.qmm_pack_swiglu((w2, s2, s2), (w3, s3, s3), bits=8)
    pair = ops.qmm_pack_swiglu((w3, s3, s3), (w3, s3, s3), bits=8)
    with pytest.raises(ValueError):                       # x with the wrong K
        ops.quantized_swiglu_packed(torch.zeros((4, 1024), dtype=torch.bfloat16, device=dev), pair)
