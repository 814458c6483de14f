"""GPU: the host mirror routes real calls through the kernels and matches the oracle / the stock
path under the reference's own contracts:

- small_m_matmul: inside the window the kernel serves the call, within
  ``0.02 * max(max|stock|, 1)`` of the stock path (small_m_qmm.py:120); outside it the result
  is the stock path bit for bit (tests/test_small_m_qmm.py:94-104);
- multirow_attention: an eligible causal / tree call equals the oracle within the attention tolerance;
  an ineligible call falls through unchanged (multirow_attn.py:338-370);
- gather_qmm / SwitchGLU / SparseMoeBlock against the MoE oracle (sorted and unsorted pairs).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import assert_rms_close, from_dev_bf16
from oracle import attn_ref, moe_ref

pytestmark = pytest.mark.gpu


def _ql(dev, bits, n, k, seed, bias=False):
    from dspark_rocm.nn import QuantizedLinear

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return QuantizedLinear.random(n, k, bits=bits, device=dev, generator=g, bias=bias)


@pytest.mark.parametrize("bits", [4, 8])
def test_small_m_scope_serves_window_and_stock_outside(dev, bits):
    from dspark_rocm import small_m_qmm as sm

    mod = _ql(dev, bits, 512, 1024, 7, bias=True)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    for m in (1, 5, 8, 12, 16, 17, 32):
        x = (torch.randn((m, 1024), generator=g, device=dev) * 0.1).to(torch.bfloat16)
        stock = mod.stock(x)
        with sm.small_m_matmul(frozenset({id(mod)})):
            got = mod(x)
            assert sm.serves(mod, x) == (m <= 16)
        if m <= 16:
            ref = stock.float()
            assert (got.float() - ref).abs().max().item() <= 0.02 * max(ref.abs().max().item(), 1.0), m
            # the kernel path is what ran: equal to a direct kernel call plus the bias
            direct = sm._kernel_rows(mod, x) + mod.bias
            assert torch.equal(got, direct)
        else:
            assert torch.equal(got, stock), m


def test_small_m_leading_dims_and_numerics_gate(dev):
    from dspark_rocm import skinny_qmm as sk
    from dspark_rocm import small_m_qmm as sm

    mod = _ql(dev, 4, 256, 512, 3)
    x = torch.randn((2, 3, 512), device=dev).to(torch.bfloat16)
    with sm.small_m_matmul(frozenset({id(mod)})):
        y = mod(x)
    assert y.shape == (2, 3, 256)
    assert torch.equal(y.reshape(6, 256), sk.qmm(x.reshape(6, 512), mod.weight, mod.scales, mod.biases, 4))
    assert sm.numerics_ok(mod)


def test_small_m_gate_verdicts(dev, monkeypatch):
    """The gate returns a shape exactly when numerics pass and every race bar is met: a race the
    kernel wins enables the shape, one bar missed disables it, a kernel output that drifts from
    the stock path disables it whatever the race says."""
    from dspark_rocm import small_m_qmm as sm

    mods = torch.nn.ModuleList([_ql(dev, 4, 256, 512, 3), _ql(dev, 4, 256, 512, 4), _ql(dev, 8, 128, 512, 5)])
    key4, key8 = sm.shape_key(mods[0]), sm.shape_key(mods[2])
    seen = []

    def race(ratio_at):
        def fake(ms, rows, gen):
            seen.append((sm.shape_key(ms[0]), rows, len(ms)))
            return ratio_at(rows)
        return fake

    monkeypatch.setattr(sm, "_race", race(lambda rows: 2.0))
    assert sorted(sm.measure_shapes(mods)) == sorted([key4, key8])
    # both 4-bit modules race together; the window starts at M = 1 < 6, so the edge bar is raced
    assert (key4, 8, 2) in seen and (key4, 12, 2) in seen and (key4, 1, 2) in seen
    monkeypatch.setattr(sm, "_race", race(lambda rows: 1.10 if rows == 12 else 2.0))     # M = 12 below 1.15
    assert sm.measure_shapes(mods) == []
    monkeypatch.setattr(sm, "_race", race(lambda rows: 0.96 if rows == 1 else 2.0))      # edge below 0.97
    assert sm.measure_shapes(mods) == []
    monkeypatch.setattr(sm, "_race", race(lambda rows: 0.97 if rows == 1 else 1.15))     # every bar met exactly
    assert len(sm.measure_shapes(mods)) == 2
    monkeypatch.setattr(sm, "_race", race(lambda rows: 2.0))
    real = sm._kernel_rows
    monkeypatch.setattr(sm, "_kernel_rows", lambda mod, x: real(mod, x) * 1.05 + 0.5)    # drifted kernel
    assert sm.measure_shapes(mods) == []


def test_small_m_gate_enables_a_real_shape(dev):
    """The real race on an 8B-shaped projection (4096 x 4096, 8-bit, four layers): the kernel
    must clear the reference's bars (1.15x at M = 8 and 12, 0.97x at M = 1) against the stock
    dequantize-and-matmul path on this GPU."""
    from dspark_rocm import small_m_qmm as sm

    mods = torch.nn.ModuleList([_ql(dev, 8, 4096, 4096, 20 + i) for i in range(4)])
    assert sm.measure_shapes(mods, verbose=True) == [sm.shape_key(mods[0])]


def _kv(dev, hk, L, d, seed, cap_extra=32):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    kb = torch.randn((1, hk, L + cap_extra, d), generator=g, device=dev).to(torch.bfloat16)
    vb = torch.randn((1, hk, L + cap_extra, d), generator=g, device=dev).to(torch.bfloat16)
    return kb[:, :, :L], vb[:, :, :L]          # cache views with capacity > L


def _np(t):
    return t.float().cpu().numpy().astype(np.float64)


def test_multirow_scope_routes_causal_tree_and_falls_through(dev):
    from dspark_rocm import fast, multirow_attn as mra

    hq, hk, d, ql, L = 32, 8, 128, 8, 2048
    cfg = mra.MultirowConfig((mra.Window(hq, hk, d, min_q=2, max_q=16, min_kv=1024),))
    k, v = _kv(dev, hk, L, d, 11)
    q = torch.randn((1, hq, ql, d), device=dev).to(torch.bfloat16)
    scale = d ** -0.5
    ref = attn_ref.attention(_np(q), _np(k), _np(v), scale, True)
    with mra.multirow_attention(cfg):
        out = fast.scaled_dot_product_attention(q, k, v, scale=scale, mask="causal")
        assert_rms_close(_np(out), ref, 2e-2, "scope causal")
        assert torch.equal(out, mra.multirow_sdpa(q, k, v, scale=scale, causal=True))
        # tree verify: the registered mask object takes the ancestry variant
        anc = torch.tensor([(1 << (i + 1)) - 1 if i % 3 else 1 << i for i in range(ql)], dtype=torch.int32)
        tmask = object()
        with mra.tree_mask(tmask, anc.to(dev)):
            tout = fast.scaled_dot_product_attention(q, k, v, scale=scale, mask=tmask)
        tref = attn_ref.attention(_np(q), _np(k), _np(v), scale, causal=False, tree_anc=anc.numpy())
        assert_rms_close(_np(tout), tref, 2e-2, "scope tree")
        # an array mask is not eligible: the stock path runs, unchanged
        amask = torch.ones((ql, L), dtype=torch.bool, device=dev)
        fell = fast.scaled_dot_product_attention(q, k, v, scale=scale, mask=amask)
        assert torch.equal(fell, fast.STOCK(q, k, v, scale=scale, mask=amask))
        # a short cache is below the window's min_kv: stock too
        ks, vs = k[:, :, :512], v[:, :, :512]
        assert torch.equal(fast.scaled_dot_product_attention(q, ks, vs, scale=scale, mask="causal"),
                           fast.STOCK(q, ks, vs, scale=scale, mask="causal"))


def test_measure_window_finds_the_kernel_window(dev):
    from dspark_rocm import multirow_attn as mra

    window, report = mra.measure_window(32, 8, 128, probe_q=(2, 4, 8, 16), probe_kv=(1024, 4096))
    assert "reason" not in report or window is not None, report
    assert window is not None and window["max_q"] >= 8, report


def _moe_weights(dev, E, H, I, bits, seed):
    from dspark_rocm.moe import SwitchGLU

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return SwitchGLU.random(E, H, I, bits=bits, device=dev, generator=g)


def _host(lin):
    w, s, b = lin.triple()
    return w.cpu().numpy().view(np.uint32), from_dev_bf16(s), from_dev_bf16(b)


@pytest.mark.parametrize("sorted_pairs", [False, True])
def test_gather_qmm_matches_oracle(dev, sorted_pairs):
    from dspark_rocm.moe import gather_qmm

    E, H, I, bits = 8, 256, 128, 4
    mlp = _moe_weights(dev, E, H, I, bits, 2)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    x = torch.randn((6, 1, H), generator=g, device=dev).to(torch.bfloat16)
    experts = torch.randint(0, E, (6,), generator=g, device=dev)
    if sorted_pairs:
        experts, _ = torch.sort(experts)
    y = gather_qmm(x, *mlp.gate_proj.triple(), rhs_indices=experts, bits=bits, sorted_indices=sorted_pairs)
    assert y.shape == (6, 1, I)
    w, s, b = _host(mlp.gate_proj)
    ref = moe_ref.gather_qmm(_np(x.reshape(6, H)), list(range(6)), experts.cpu().tolist(), w, s, b, bits)
    assert_rms_close(_np(y.reshape(6, I)), ref, 2e-2, "gather_qmm")


@pytest.mark.parametrize("M", [4, 16])                 # 4*8 = 32 pairs (unsorted), 128 (sorted)
def test_switch_glu_and_sparse_moe_block_match_oracle(dev, M):
    from dspark_rocm.moe import SparseMoeBlock, route
    from dspark_rocm.nn import QuantizedLinear

    E, H, I, k, bits = 32, 256, 128, 8, 4
    mlp = _moe_weights(dev, E, H, I, bits, 5)
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    router = QuantizedLinear.random(E, H, bits=8, device=dev, generator=g)
    block = SparseMoeBlock(router, mlp, top_k=k)
    x = torch.randn((M, H), generator=g, device=dev).to(torch.bfloat16)
    logits = block.router_logits(x)
    hx, hl = _np(x), _np(logits)
    ref, rinds, _ = moe_ref.switch_glu(hx, hl, *_host(mlp.gate_proj), *_host(mlp.up_proj), *_host(mlp.down_proj),
                                       k=k, bits=bits)
    inds, scores = route(logits, k)
    assert np.array_equal(inds.cpu().numpy(), rinds)
    y = mlp(x, inds)                                   # [M, k, H] per (token, slot)
    assert y.shape == (M, k, H)
    fused = block(x)
    unfused = block.forward_unfused(x)
    assert_rms_close(_np(fused), ref, 2e-2, "SparseMoeBlock fused")
    assert_rms_close(_np(unfused), ref, 2e-2, "SparseMoeBlock unfused")


def test_apply_wiring_measures_and_routes(dev, tmp_path, monkeypatch):
    """The load-time wiring end to end on this GPU: apply_small_m and apply_multirow_attn race
    the real kernels for a model's shapes (hidden 1024, intermediate 4096, 8/2 heads x 128),
    cache the verdicts, and verify_scopes then routes the module path through the kernels; its
    logits match the fused engine's."""
    from _model_util import tiny_model

    from dspark_rocm import calibrate, multirow_attn, small_m_qmm
    from dspark_rocm.model import Target

    monkeypatch.setenv("DSPARK_CACHE_DIR", str(tmp_path))
    monkeypatch.setattr(calibrate, "SMALL_M_IDS", None)
    monkeypatch.setattr(calibrate, "MULTIROW_CFG", None)
    model = tiny_model(dev, seed=12, hidden_size=1024, intermediate_size=4096, num_attention_heads=8,
                       num_key_value_heads=2)
    ids = calibrate.apply_small_m(model, target_repo="synthetic-1024", verbose=True)
    cfg = calibrate.apply_multirow_attn(model, verbose=True)
    assert ids, "the small-M kernel should win on a 1024 x 4096 8-bit model on MI355X"
    assert cfg is not None and cfg.window(8, 2, 128) is not None
    assert len(list(tmp_path.iterdir())) >= 2                      # both verdicts cached
    tgt = Target(model)
    ids_t = torch.tensor([[7, 1, 8, 2, 8, 1, 8, 2, 8, 4, 5, 9, 0, 4, 5, 2]])
    fused, _ = tgt.verify(ids_t, tgt.make_cache(64))
    cb = tgt.make_cache(64)
    with calibrate.verify_scopes(), torch.no_grad():
        assert small_m_qmm.active() and multirow_attn.active()
        mod = model(ids_t.to(dev), cb)
    assert_rms_close(_np(mod[0]), _np(fused[0]), 5e-2, "module path under the applied scopes vs fused")
