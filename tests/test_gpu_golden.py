"""GPU: the kernels against the committed golden fixtures (tests/golden/): routing indices,
score bits and bucketing bit-exact; qmm, attention (causal and tree) and the grouped qmm within
max|d| <= 2e-2 * RMS of the fixture."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from _util import assert_rms_close, from_dev_bf16, to_dev_packed
from oracle import quant_ref

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, f"{name}.npz"))


def _bits_to_dev(bits16, dev):
    return torch.from_numpy(np.ascontiguousarray(bits16).view(np.int16).copy()).to(dev).view(torch.bfloat16)


@pytest.mark.parametrize("bits", [4, 8])
def test_qmm_golden(dev, bits):
    from dspark_rocm import ops

    f = _load("qmm")
    w, s, b = to_dev_packed(f[f"w{bits}"], dev), _bits_to_dev(f[f"s{bits}"], dev), _bits_to_dev(f[f"b{bits}"], dev)
    for m in (1, 5, 8, 16):
        y = ops.quantized_matmul(_bits_to_dev(f[f"x{bits}_{m}"], dev), w, s, b, bits=bits)
        assert_rms_close(from_dev_bf16(y), f[f"y{bits}_{m}"], 2e-2, f"qmm {bits}-bit M={m}")


def test_attention_golden(dev):
    from dspark_rocm import ops

    f = _load("attention")
    anc = torch.from_numpy(f["tree_anc"].astype(np.int64)).to(torch.int32)
    for L in (48, 300):
        q, k, v = (_bits_to_dev(f[f"{t}{L}"], dev) for t in "qkv")
        out = ops.verify_attention(q, k, v, scale=128 ** -0.5, causal=True)
        assert_rms_close(from_dev_bf16(out), f[f"causal{L}"], 2e-2, f"causal L={L}")
        out = ops.verify_attention(q, k, v, scale=128 ** -0.5, causal=False, tree_anc=anc)
        assert_rms_close(from_dev_bf16(out), f[f"tree{L}"], 2e-2, f"tree L={L}")


def test_route_golden_bit_exact(dev):
    from dspark_rocm import ops

    f = _load("route")
    inds, scores, off, srt, pos = ops.moe_route(_bits_to_dev(f["logits"], dev), 8, bucket=True)
    assert np.array_equal(inds.cpu().numpy(), f["inds"])
    assert np.array_equal(scores.view(torch.int16).cpu().numpy().view(np.uint16), f["scores"])
    assert np.array_equal(off.cpu().numpy(), f["offsets"])
    assert np.array_equal(srt.cpu().numpy(), f["sorted"])
    assert np.array_equal(pos.cpu().numpy(), f["pos"])


def test_gather_qmm_golden(dev):
    from dspark_rocm.moe import gather_qmm

    f = _load("gather_qmm")
    x = _bits_to_dev(f["x"], dev)
    w = to_dev_packed(f["w"].reshape(-1, f["w"].shape[-1]), dev).view(f["w"].shape)
    s, b = _bits_to_dev(f["s"], dev), _bits_to_dev(f["b"], dev)
    inds = torch.from_numpy(f["inds"].astype(np.int64)).to(dev)
    y = gather_qmm(x.unsqueeze(1).unsqueeze(1), w, s, b, rhs_indices=inds, bits=4)    # [6, 2, 1, 64]
    assert_rms_close(from_dev_bf16(y.reshape(12, 64)), quant_ref.bf16_from_bits(f["y"]), 2e-2, "gather_qmm")
