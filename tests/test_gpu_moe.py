"""GPU parity of MoE routing, bucketing, gather_qmm and the fused SwitchGLU block.

Routing indices, bucket offsets and the sorted pair order must be bit-exact against the oracle
(the order rule is documented in oracle/moe_ref.py); scores within one bf16 ulp; expert outputs
within 2e-2 * RMS. mlx-lm's own MoE code is not in the reference tree, so the oracle is pinned
by brute force (tests/test_oracle_moe.py).
"""

from __future__ import annotations

import numpy as np
import pytest

from _util import assert_rms_close, from_dev_bf16, randn_bf16, rng, to_dev_bf16, to_dev_packed
from oracle import moe_ref, quant_ref

pytestmark = pytest.mark.gpu


def _logits_with_ties(r, M, E):
    x = randn_bf16(r, M, E)
    # deliberate exact ties (same bf16 logit) inside and across the top-k boundary
    x[0, 5] = x[0, 9] = x[0, E - 3] = x[0].max()
    x[1, :16] = 2.0
    x[2, E // 2:] = x[2].max()
    x[3, :] = 0.0
    return x


@pytest.mark.parametrize("M,E,k", [(16, 128, 8), (1, 128, 8), (4, 64, 4), (16, 256, 8), (33, 128, 2),
                                   (65, 128, 8), (200, 64, 4), (1024, 128, 8), (97, 512, 3), (256, 1024, 32)])
def test_route_bit_exact(dev, M, E, k):
    import torch

    from dspark_rocm import ops

    r = rng(M * 1000 + E + k)
    x = _logits_with_ties(r, M, E) if M >= 4 else randn_bf16(r, M, E)
    inds, scores, off, srt, pos = ops.moe_route(to_dev_bf16(x, dev), k, bucket=True)
    ri, rs = moe_ref.route(x, k)
    assert np.array_equal(inds.cpu().numpy(), ri)
    got_s = from_dev_bf16(scores)
    ulp = np.abs(rs) * 2.0 ** -7
    assert np.all(np.abs(got_s - rs) <= ulp + 1e-9), np.max(np.abs(got_s - rs))
    ro, rsrt, rpos = moe_ref.bucket(ri, E)
    assert np.array_equal(off.cpu().numpy(), ro)
    assert np.array_equal(srt.cpu().numpy(), rsrt)
    assert np.array_equal(pos.cpu().numpy(), rpos)
    assert torch.all(inds >= 0) and torch.all(inds < E)


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_qmm(dev, bits):
    import torch

    from dspark_rocm import ops

    r = rng(20 + bits)
    E, N, K, P = 8, 96, 256, 40
    experts = np.sort(r.integers(0, E, size=P)).astype(np.int32)
    experts[experts == 3] = 4                      # an empty expert
    experts = np.sort(experts)
    rows = r.integers(0, 12, size=P).astype(np.int32)
    x = randn_bf16(r, 12, K)
    mats = [quant_ref.random_packed(r, N, K, bits) for _ in range(E)]
    w = np.stack([m[0] for m in mats])
    s = np.stack([m[1] for m in mats])
    b = np.stack([m[2] for m in mats])
    offsets = np.concatenate([[0], np.cumsum(np.bincount(experts, minlength=E))]).astype(np.int32)
    y = ops.gather_qmm_sorted(to_dev_bf16(x, dev), to_dev_packed(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev),
                              torch.from_numpy(offsets).to(dev), row_index=torch.from_numpy(rows).to(dev), bits=bits)
    ref = moe_ref.gather_qmm(x, rows, experts, w, s, b, bits)
    assert_rms_close(from_dev_bf16(y), ref, 2e-2, "gather_qmm")


def _moe_weights(r, E, H, I, bits):
    def stack(n, k):
        mats = [quant_ref.random_packed(r, n, k, bits) for _ in range(E)]
        return tuple(np.stack([m[i] for m in mats]) for i in range(3))
    return stack(I, H), stack(I, H), stack(H, I)


def _dev3(t, dev):
    return to_dev_packed(t[0], dev), to_dev_bf16(t[1], dev), to_dev_bf16(t[2], dev)


@pytest.mark.parametrize("M,E,k,H,I,bits", [(16, 8, 2, 256, 128, 4), (5, 16, 4, 512, 192, 8),
                                             (16, 128, 8, 2048, 768, 4),
                                             (16, 128, 8, 2048, 768, 8),  # the A3B block with 8-bit experts
                                             (16, 2, 2, 512, 256, 4),     # every token in both experts: 16-row buckets
                                             (33, 4, 2, 256, 4096, 8)])   # 3 row tiles; down K = 4096 in 4 K parts
def test_switch_glu(dev, M, E, k, H, I, bits):
    from dspark_rocm import ops

    r = rng(M + E + H)
    x = randn_bf16(r, M, H)
    logits = randn_bf16(r, M, E)
    g, u, d = _moe_weights(r, E, H, I, bits)
    out, inds, scores = ops.moe_switch_glu(to_dev_bf16(x, dev), to_dev_bf16(logits, dev), _dev3(g, dev),
                                           _dev3(u, dev), _dev3(d, dev), k=k, bits=bits)
    ref, ri, rs = moe_ref.switch_glu(x, logits, *g, *u, *d, k=k, bits=bits)
    assert np.array_equal(inds.cpu().numpy(), ri)
    assert_rms_close(from_dev_bf16(out), ref, 2e-2, "switch_glu")
    # a second call gives the same bits (the combine's arrival counters were left at zero)
    out2, _, _ = ops.moe_switch_glu(to_dev_bf16(x, dev), to_dev_bf16(logits, dev), _dev3(g, dev), _dev3(u, dev),
                                    _dev3(d, dev), k=k, bits=bits)
    import torch

    assert torch.equal(out2, out)


@pytest.mark.parametrize("M,E,k,H,I,bits", [(16, 8, 2, 256, 128, 4), (16, 128, 8, 2048, 768, 4),
                                             (16, 128, 8, 2048, 768, 8), (16, 2, 2, 512, 256, 4),
                                             (16, 2, 2, 512, 256, 8),
                                             (1, 128, 8, 2048, 768, 4),     # 8 one-row buckets
                                             (5, 128, 8, 2048, 768, 8),
                                             (16, 256, 8, 2048, 768, 4),    # E = 256: four ballots
                                             (7, 64, 6, 512, 256, 4),
                                             (33, 4, 2, 256, 4096, 8)])
def test_switch_glu_packed_experts_bitwise(dev, M, E, k, H, I, bits):
    """The packed expert form (dspark_moe_pack) gives the row-major block's output bit for bit
    (same K parts, same per-group arithmetic and order), and its bytes are the weight part of the
    dense packed layout of each expert's matrix. For M <= 16 and H in {512, 2048} the packed
    block's gate/up runs one workgroup per CU (ops.moe_packed_plan) and the row-major block's one
    workgroup per (expert, strip): the two kernels agree bit for bit, 16-row buckets (E = 2) and
    one-row buckets (M = 1) included."""
    import torch

    from dspark_rocm import ops
    from test_gpu_qmm_packed import _pack_np

    plan = ops.moe_packed_plan(M, H, I, E, k, bits)
    assert plan["gate_up"] == ("per CU" if M <= 16 and H in (512, 2048) else "expert x strip")

    r = rng(M + E + H + 1)
    x = to_dev_bf16(randn_bf16(r, M, H), dev)
    logits = to_dev_bf16(randn_bf16(r, M, E), dev)
    g, u, d = _moe_weights(r, E, H, I, bits)
    rm = [_dev3(t, dev) for t in (g, u, d)]
    pk = [(ops.moe_pack(w, bits=bits), s, b) for (w, s, b) in rm]
    out, inds, scores = ops.moe_switch_glu(x, logits, *rm, k=k, bits=bits)
    out_p, inds_p, scores_p = ops.moe_switch_glu(x, logits, *pk, k=k, bits=bits)
    assert torch.equal(inds_p, inds) and torch.equal(scores_p, scores)
    assert torch.equal(out_p, out)
    # layout: expert e's bytes are the weight tiles of its [n, kk] matrix in the dense packed form
    w, s, b = d
    n, kk = w.shape[1], w.shape[2] * 32 // bits
    got = pk[2][0].buf.cpu().numpy().reshape(E, -1)
    wbytes = got.shape[1]
    for e in (0, E - 1):
        assert np.array_equal(got[e], _pack_np(w[e], s[e], b[e], n, kk, bits)[:wbytes])


def test_moe_pack_refusals(dev):
    import torch

    from dspark_rocm import _lib, ops

    assert ops.moe_packable(4, 768, 2048, 4) and not ops.moe_packable(4, 760, 2048, 4)   # N % 16
    assert not ops.moe_packable(4, 2048, 192, 8)                                          # K % 128
    w = torch.zeros((4, 2048, 192 // 4), dtype=torch.int32, device=dev)
    with pytest.raises(_lib.DsparkError):
        ops.moe_pack(w, bits=8)
