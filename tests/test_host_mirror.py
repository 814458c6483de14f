"""CPU tests of the host-side mirror of the reference's kernel call surface: launch plans,
scopes (install / restore / nest / fall through), eligibility gates, the row-split fallback,
the stock attention path against the oracle, byte accounting. No kernel is launched.

Structure follows the reference's tests: tests/test_sdpa_split.py:50-74,
tests/test_multirow_attn.py:102-109, tests/test_small_m_qmm.py:94-171 and :250-260,
tests/test_roofline.py:40-80.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attn_ref


# ---------------------------------------------------------------- sdpa_split

def test_partition_sums_and_bounds():
    from dspark_rocm.sdpa_split import _partition

    for q in range(1, 33):
        parts = _partition(q, 5)
        assert sum(parts) == q
        assert all(1 <= p <= 5 for p in parts)
        assert max(parts) - min(parts) <= 1
        assert parts == sorted(parts, reverse=True)
    assert _partition(12, 5) == [4, 4, 4] and _partition(7, 5) == [4, 3] and _partition(5, 5) == [5]


def _qkv(qlen, L, hq=4, hk=2, d=32, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((1, hq, qlen, d), generator=g).to(dtype)
    k = torch.randn((1, hk, L, d), generator=g).to(dtype)
    v = torch.randn((1, hk, L, d), generator=g).to(dtype)
    return q, k, v


@pytest.mark.parametrize("mask", ["causal", "arr", None])
@pytest.mark.parametrize("qlen", [6, 7, 8, 12])
def test_split_equals_single_when_firing(mask, qlen):
    from dspark_rocm import fast
    from dspark_rocm.sdpa_split import SplitConfig, split_sdpa

    cfg = SplitConfig(min_q=6, max_q=15, min_kv=64, max_chunk=5)
    q, k, v = _qkv(qlen, 200)
    m = mask
    if mask == "arr":
        g = torch.Generator().manual_seed(5)
        m = torch.rand((1, 1, qlen, 200), generator=g) > 0.3
        m[..., 0] = True
    single = fast.STOCK(q, k, v, scale=0.2, mask=m)
    split = split_sdpa(q, k, v, scale=0.2, mask=m, cfg=cfg)
    assert split.shape == single.shape
    assert (split - single).abs().max().item() < 1e-5


@pytest.mark.parametrize("qlen,L", [(1, 512), (4, 512), (8, 32)])
def test_split_gate_passthrough_is_bit_identical(qlen, L):
    from dspark_rocm import fast
    from dspark_rocm.sdpa_split import SplitConfig, split_sdpa

    cfg = SplitConfig(min_q=6, max_q=15, min_kv=64, max_chunk=5)
    q, k, v = _qkv(qlen, L)
    assert torch.equal(fast.STOCK(q, k, v, scale=0.2, mask="causal"),
                       split_sdpa(q, k, v, scale=0.2, mask="causal", cfg=cfg))


def test_split_scope_installs_and_restores():
    from dspark_rocm import fast, sdpa_split

    stock = fast.scaled_dot_product_attention
    with sdpa_split.sdpa_split(sdpa_split.SplitConfig()):
        assert fast.scaled_dot_product_attention is sdpa_split._patched_call
        with sdpa_split.sdpa_split(sdpa_split.SplitConfig()):       # nested: no-op
            assert fast.scaled_dot_product_attention is sdpa_split._patched_call
        assert fast.scaled_dot_product_attention is sdpa_split._patched_call
    assert fast.scaled_dot_product_attention is stock
    with sdpa_split.sdpa_split(None):
        assert fast.scaled_dot_product_attention is stock
    assert sdpa_split.patchable()


# ---------------------------------------------------------------- stock attention vs the oracle

@pytest.mark.parametrize("causal", [True, False])
def test_stock_sdpa_matches_oracle(causal):
    from dspark_rocm import fast

    q, k, v = _qkv(5, 40, hq=4, hk=2, d=16, seed=3, dtype=torch.float64)
    got = fast.STOCK(q.float(), k.float(), v.float(), scale=0.25, mask="causal" if causal else None)
    ref = attn_ref.attention(q.numpy(), k.numpy(), v.numpy(), 0.25, causal)
    assert np.abs(got.double().numpy() - ref).max() < 1e-5


def test_stock_sdpa_sinks():
    """A sink logit of -inf changes nothing; a finite sink only rescales every row by
    sum(exp(s)) / (sum(exp(s)) + exp(sink)) (closed form)."""
    from dspark_rocm import fast

    q, k, v = _qkv(3, 20, hq=2, hk=2, d=8, seed=4, dtype=torch.float64)
    base = fast.STOCK(q, k, v, scale=0.5)
    none = fast.STOCK(q, k, v, scale=0.5, sinks=torch.full((2,), float("-inf"), dtype=torch.float64))
    assert torch.allclose(base, none)
    sink = torch.tensor([0.3, -1.2], dtype=torch.float64)
    got = fast.STOCK(q, k, v, scale=0.5, sinks=sink)
    s = torch.matmul(q, k.transpose(-1, -2)) * 0.5
    z = torch.exp(s).sum(-1, keepdim=True)
    factor = z / (z + torch.exp(sink).reshape(1, 2, 1, 1))
    assert torch.allclose(got, base * factor, rtol=1e-5, atol=1e-6)   # fp32 internally


# ---------------------------------------------------------------- multirow_attn

def test_multirow_plan_kats():
    from dspark_rocm import _lib
    from dspark_rocm.multirow_attn import plan

    p = plan(32, 8, 16, 128, 32784)                  # 32/8 heads at 32k: 64 rows of one KV head
    assert (p["R"], p["RP"], p["NRG"]) == (64, 64, 1)
    assert p["CHUNK"] % 64 == 0 and p["NB"] * p["CHUNK"] >= 32784 > (p["NB"] - 1) * p["CHUNK"]
    assert p["workgroups"] == 8 * p["NB"] <= 512                   # at most 2 resident 4-wave workgroups per CU
    p = plan(32, 8, 4, 128, 1024)                    # 16 rows: one row tile
    assert (p["R"], p["RP"], p["NRG"]) == (16, 16, 1)
    short = plan(32, 8, 16, 128, 64)
    assert short["NB"] == 1                          # one block: no partials
    nbs = [plan(32, 8, 16, 128, L)["NB"] for L in (528, 4112, 16400, 32784)]
    assert nbs == sorted(nbs)
    with pytest.raises(_lib.DsparkError):
        plan(64, 2, 16, 128, 32768)                  # gqa * q_len = 512 rows > 256
    with pytest.raises(_lib.DsparkError):
        plan(32, 8, 16, 100, 4096)                   # head_dim % 8 != 0
    with pytest.raises(_lib.DsparkError):
        plan(32, 8, 16, 264, 4096)                   # head_dim > 256
    assert plan(32, 8, 16, 96, 4096) == plan(32, 8, 16, 128, 4096)   # runs on the 128 instance
    assert plan(24, 4, 16, 192, 4096) == plan(24, 4, 16, 256, 4096)


CFG = None


def _cfg():
    from dspark_rocm.multirow_attn import MultirowConfig, Window

    return MultirowConfig((Window(8, 2, 64, min_q=2, max_q=16, min_kv=64),))


def _bf(*shape):
    return torch.zeros(shape, dtype=torch.bfloat16)


def test_multirow_eligibility_gate():
    from dspark_rocm.multirow_attn import eligible, eligible_shape

    cfg = _cfg()
    q, k, v = _bf(1, 8, 4, 64), _bf(1, 2, 256, 64), _bf(1, 2, 256, 64)
    assert eligible_shape(q, k, v, "causal", None, cfg)
    assert eligible_shape(q, k, v, None, None, cfg)
    assert not eligible(q, k, v, "causal", None, cfg)                     # CPU tensors: never
    assert not eligible_shape(q, k, v, "causal", torch.zeros(8), cfg)     # sinks
    assert not eligible_shape(q, k, v, torch.ones(4, 256, dtype=torch.bool), None, cfg)  # array mask
    assert not eligible_shape(_bf(1, 8, 1, 64), k, v, "causal", None, cfg)  # q_len below window
    assert not eligible_shape(_bf(1, 8, 17, 64), k, v, "causal", None, cfg)  # above window
    assert not eligible_shape(q, _bf(1, 2, 32, 64), _bf(1, 2, 32, 64), "causal", None, cfg)  # short KV
    assert not eligible_shape(_bf(1, 16, 4, 64), k, v, "causal", None, cfg)  # unmeasured shape
    assert not eligible_shape(q.float(), k.float(), v.float(), "causal", None, cfg)  # dtype
    kt = _bf(1, 2, 64, 256).transpose(-1, -2)                            # head_dim not contiguous
    assert not eligible_shape(q, kt, v, "causal", None, cfg)
    assert not eligible_shape(q, k, v, "bidirectional", None, cfg)                # unknown string mask
    kv_view = _bf(1, 2, 512, 64)[:, :, :256]                              # sequence-sliced view: fine
    assert eligible_shape(q, kv_view, kv_view, "causal", None, cfg)


def test_multirow_scope_nests_over_split_and_falls_through():
    from dspark_rocm import fast, multirow_attn, sdpa_split

    stock = fast.scaled_dot_product_attention
    with sdpa_split.sdpa_split(sdpa_split.SplitConfig(min_q=6, max_q=15, min_kv=64, max_chunk=5)):
        with multirow_attn.multirow_attention(_cfg()):
            assert multirow_attn.active()
            # CPU call: not eligible -> falls through to the split patch, then stock
            q, k, v = _qkv(8, 200, hq=8, hk=2, d=64)
            out = fast.scaled_dot_product_attention(q, k, v, scale=0.125, mask="causal")
            ref = fast.STOCK(q, k, v, scale=0.125, mask="causal")
            assert (out - ref).abs().max().item() < 1e-5
        assert fast.scaled_dot_product_attention is sdpa_split._patched_call
    assert fast.scaled_dot_product_attention is stock


def test_multirow_scope_restores_on_exception():
    from dspark_rocm import fast, multirow_attn

    stock = fast.scaled_dot_product_attention
    with pytest.raises(RuntimeError), multirow_attn.multirow_attention(_cfg()):
        raise RuntimeError("boom")
    assert fast.scaled_dot_product_attention is stock and not multirow_attn.active()


def test_window_from_wins():
    """The served window: the longest run of winning q (from the smallest probe) at the deepest
    kv, and the shortest kv from which every deeper probe wins that run."""
    from dspark_rocm.multirow_attn import _window_from_wins

    q, kv = (2, 4, 6, 8, 12, 16), (1024, 4096, 16384)
    assert _window_from_wins({16384: {2, 4, 6, 8}, 4096: {2, 4, 6, 8, 12}, 1024: {2, 4}}, q, kv) == \
        {"min_q": 2, "max_q": 8, "min_kv": 4096}
    assert _window_from_wins({16384: set(q), 4096: set(q), 1024: set(q)}, q, kv)["min_kv"] == 1024
    assert _window_from_wins({16384: {4, 6}}, q, kv) is None            # q = 2 lost: no run
    assert _window_from_wins({16384: {2, 6}, 4096: {2}}, q, kv) == {"min_q": 2, "max_q": 2, "min_kv": 4096}
    assert _window_from_wins({16384: {2}, 4096: set(), 1024: {2}}, q, kv)["min_kv"] == 16384


def test_tree_mask_scope_is_identity_matched_and_restored():
    from dspark_rocm import multirow_attn

    m1, m2 = torch.ones(2, 2, dtype=torch.bool), torch.ones(2, 2, dtype=torch.bool)
    with multirow_attn.tree_mask(m1, torch.tensor([1, 3], dtype=torch.int32)):
        assert multirow_attn.current_tree()[0] is m1
        with multirow_attn.tree_mask(m2, torch.tensor([1, 3], dtype=torch.int32)):
            assert multirow_attn.current_tree()[0] is m2
        assert multirow_attn.current_tree()[0] is m1
    assert multirow_attn.current_tree() is None


# ---------------------------------------------------------------- skinny_qmm / small_m_qmm

def test_skinny_plan_geometry():
    from dspark_rocm import skinny_qmm as sk

    for n, k in ((4096, 4096), (24576, 4096), (4096, 12288), (1024, 4096), (64, 4096), (1024, 1024)):
        p = sk.plan(16, n, k, 8)
        assert p["strips"] == -(-n // 64)
        if (n, k) == (4096, 4096):
            # 8-bit [4096, 4096]: one 16-row workgroup per tile over all of K, no workspace
            assert (p["slices"], p["groups_per_slice"], p["workgroups"]) == (1, 64, 256)
        else:
            assert p["workgroups"] == p["slices"] * p["strips"]
            assert p["groups_per_slice"] in (8, 16, 32)
        assert p["slices"] * p["groups_per_slice"] >= k // 64
        assert (p["workspace_bytes"] > 0) == (p["slices"] > 1)
        assert p | {"rows": 5} == sk.plan(5, n, k, 8)   # the plan does not depend on M (<= 16)
        assert sk.plan(33, n, k, 8)["slices"] == p["slices"]   # nor does the kernel choice, at any M
    # the same K split serves 4 and 8 bits, and so does the whole-K launch of [4096, 4096]
    assert sk.plan(16, 4096, 12288, 4)["slices"] == sk.plan(16, 4096, 12288, 8)["slices"]
    p4 = sk.plan(16, 4096, 4096, 4)
    assert (p4["slices"], p4["groups_per_slice"], p4["workgroups"], p4["workspace_bytes"]) == (1, 64, 256, 0)
    assert sk.plan(16, 4096, 2048, 4)["slices"] > 1   # K = 2048 keeps split-K at both widths
    assert sk.geometry(4096, 4096) == (64, 1)
    assert sk.geometry(4096, 4096, bits=4) == (64, 1)


def _qlinear(bits=4, out_features=64, in_features=128, bias=False):
    from dspark_rocm.nn import QuantizedLinear

    g = torch.Generator().manual_seed(bits + out_features)
    return QuantizedLinear.random(out_features, in_features, bits=bits, generator=g, bias=bias)


def test_fits_and_shape_key():
    from dspark_rocm import skinny_qmm as sk
    from dspark_rocm.small_m_qmm import eligible, shape_key

    a, b = _qlinear(4), _qlinear(8)
    assert sk.fits(a) and sk.fits(b) and eligible(a)
    assert shape_key(a) != shape_key(b) and shape_key(a) == "128x64b4"
    b.scales = b.scales.float()
    assert not sk.fits(b)
    assert not eligible(torch.nn.Linear(4, 4))


def test_dispatch_window_and_allowlist():
    from dspark_rocm import small_m_qmm as sm

    mod, other = _qlinear(4), _qlinear(8)
    x = torch.zeros((4, 2, 128), dtype=torch.bfloat16)          # M = 8 rows
    assert not sm.serves(mod, x)                                 # scope inactive
    with sm.small_m_matmul(frozenset({id(mod)})):
        assert sm.active()
        assert sm.serves(mod, x)
        assert not sm.serves(other, torch.zeros((8, 128), dtype=torch.bfloat16))   # not listed
        assert not sm.serves(mod, x.float())                                         # not bf16
        assert not sm.serves(mod, torch.zeros((17, 128), dtype=torch.bfloat16))    # above window
        assert sm.serves(mod, torch.zeros((1, 128), dtype=torch.bfloat16))         # M = 1 served
        # on the CPU every call is the stock path, bit for bit
        xx = torch.randn((8, 128), generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
        assert torch.equal(mod(xx), mod.stock(xx))
    assert not sm.active()


def test_small_m_scope_restores_and_nests():
    from dspark_rocm import small_m_qmm as sm
    from dspark_rocm.nn import QuantizedLinear

    orig = QuantizedLinear.forward
    with pytest.raises(RuntimeError), sm.small_m_matmul(frozenset({1})):
        raise RuntimeError("boom")
    assert QuantizedLinear.forward is orig and not sm.active()

    def other_scope_forward(self, x):       # another scope holding the class inside ours
        return orig(self, x)

    with sm.small_m_matmul(frozenset({1})):
        prev = QuantizedLinear.forward
        QuantizedLinear.forward = other_scope_forward
        assert not sm.active()
        QuantizedLinear.forward = prev
        assert sm.active()
    assert QuantizedLinear.forward is orig
    with sm.small_m_matmul(frozenset()):
        assert not sm.active()


def test_ids_for_shapes():
    from dspark_rocm import small_m_qmm as sm

    class Tiny(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.a, self.b, self.c = _qlinear(4), _qlinear(4), _qlinear(8)

    m = Tiny()
    ids = sm.ids_for_shapes([sm.shape_key(m.a)], m)
    assert ids == frozenset({id(m.a), id(m.b)})


def test_stock_qlinear_matches_dequant_oracle():
    from oracle import qmm_ref, quant_ref

    mod = _qlinear(8, out_features=32, in_features=256, bias=True)
    x = torch.randn((3, 256), generator=torch.Generator().manual_seed(1))
    y = mod(x).double().numpy()
    w = mod.weight.numpy().view(np.uint32)
    ref = qmm_ref.qmm_f64(x.numpy(), w, mod.scales.float().numpy(), mod.biases.float().numpy(), 8)
    ref = ref + mod.bias.float().numpy()
    assert np.abs(y - ref).max() < 1e-4 * max(1.0, np.abs(ref).max())
    assert quant_ref is not None


# ---------------------------------------------------------------- MoE host logic

def test_gather_sort_orders_pairs_by_expert():
    from dspark_rocm.moe import _gather_sort

    inds = torch.tensor([[3, 1], [1, 0], [3, 2]])
    x = torch.arange(3 * 4, dtype=torch.float32).reshape(3, 1, 1, 4)
    xs, idx, inv = _gather_sort(x, inds)
    assert idx.tolist() == [0, 1, 1, 2, 3, 3]
    pairs = torch.arange(6)[torch.sort(inds.reshape(-1), stable=True).indices]
    assert torch.equal(xs[:, 0], x.reshape(3, 4)[pairs // 2])
    assert torch.equal(idx[inv], inds.reshape(-1))


# ---------------------------------------------------------------- roofline (tests/test_roofline.py)

def test_roofline_dense_footprint():
    from dspark_rocm import roofline as R

    params = [("model.embed_tokens.weight", 1000), ("model.layers.0.mlp.weight", 5000), ("lm_head.weight", 1000)]
    fp = R.weight_footprint(params, {})
    assert fp["total_bytes"] == 7000 and fp["active_bytes"] == 6000
    assert fp["is_moe"] is False and fp["active_is_estimate"] is False


def test_roofline_tied_embeddings_count_once():
    from dspark_rocm import roofline as R

    fp = R.weight_footprint([("model.embed_tokens.weight", 1000), ("model.layers.0.mlp.weight", 5000)], {})
    assert fp["active_bytes"] == 6000


def test_roofline_moe_active_is_top_k_over_n():
    from dspark_rocm import roofline as R

    params = [("model.layers.0.mlp.switch_mlp.up_proj.weight", 1000),
              ("model.layers.0.mlp.shared_expert.up_proj.weight", 100),
              ("model.layers.0.self_attn.q_proj.weight", 50), ("lm_head.weight", 10)]
    fp = R.weight_footprint(params, {"num_experts": 100, "num_experts_per_tok": 10})
    assert fp["is_moe"] and fp["n_experts"] == 100 and fp["experts_per_tok"] == 10
    assert fp["active_bytes"] == 100 + 100 + 50 + 10 and not fp["active_is_estimate"]
    fp = R.weight_footprint(params, {"num_experts": 100})
    assert fp["active_bytes"] == 1000 + 100 + 50 + 10 and fp["active_is_estimate"]


def test_roofline_math():
    from dspark_rocm import roofline as R

    assert R.bytes_per_token(1000, 10, 50) == 1500
    assert R.ceiling_tps(None, 10) is None and R.ceiling_tps(1.0, 1_000_000_000) == 1.0
    mbu = R.baseline_mbu(2.0, 8_000_000_000, 8000.0)
    assert mbu["achieved_gb_s"] == 4000.0 and mbu["mbu"] == 0.5
    assert R.baseline_mbu(0, 1, 1.0) is None
    # the byte formulas the bench quotes (the single 4096² qmm, 32k verify attention, the A3B MoE block)
    assert R.qmm_bytes(4096, 4096, 4, 16) == 9_699_328
    assert R.qmm_bytes(4096, 4096, 8, 16) == 18_087_936
    assert R.attention_bytes(32, 8, 128, 16, 32768 + 16) == 4096 * (32768 + 16) + 262_144
    assert R.moe_bytes(1, 2048, 768, 4, 16, 128) == 2_654_208 + 135_168
    assert R.kv_bytes_per_token(64, 8, 128) == 64 * 4096


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 (or a WORLD_SIZE above 1) exits with a message
    before touching a device."""
    import json
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in json.loads(r.stdout.strip().splitlines()[-1])["error"]
