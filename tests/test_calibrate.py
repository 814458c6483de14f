"""CPU tests of the load-time wiring (dspark_rocm.calibrate): the verdict cache, the small-M
allowlist and the multi-row windows for a loaded model (measurements monkeypatched; the real
races run in the GPU tests), the stale-cache re-measure, the drafter shape probe, and the scope
order of verify_scopes (the reference's calibrate.py:1062-1153, :1352-1407, generate.py:52-83)."""

from __future__ import annotations

import pytest
import torch

from _model_util import tiny_model


@pytest.fixture
def cal(tmp_path, monkeypatch):
    from dspark_rocm import calibrate

    monkeypatch.setattr(calibrate, "SMALL_M_IDS", None)
    monkeypatch.setattr(calibrate, "MULTIROW_CFG", None)
    monkeypatch.setattr(calibrate, "SDPA_SPLIT_CFG", None)
    monkeypatch.setenv("DSPARK_CACHE_DIR", str(tmp_path))
    return calibrate


def test_cache_round_trip_and_key_check(cal, tmp_path):
    assert cal.load_cached("k1") is None
    cal.save_cached("k1", {"a": [1, 2]})
    assert cal.load_cached("k1") == {"a": [1, 2]}
    assert cal.load_cached("k2") is None
    cal.save_cached("k1", [3])
    assert cal.load_cached("k1") == [3]
    assert cal.cache_dir() == str(tmp_path)


def test_small_m_shapes_measured_once_then_cached(cal, monkeypatch):
    from dspark_rocm import small_m_qmm

    model = tiny_model("cpu", seed=1)
    calls = []

    def fake(*models, verbose=False):
        calls.append(len(models))
        return sorted({small_m_qmm.shape_key(m) for m in models[0].modules() if small_m_qmm.eligible(m)})[:2]

    monkeypatch.setattr(small_m_qmm, "measure_shapes", fake)
    a = cal.small_m_qmm_shapes(model, target_repo="t", verbose=False)
    b = cal.small_m_qmm_shapes(model, target_repo="t", verbose=False)
    assert a == b and len(a) == 2 and len(calls) == 1
    cal.small_m_qmm_shapes(model, target_repo="t", refresh=True, verbose=False)
    assert len(calls) == 2
    cal.small_m_qmm_shapes(model, target_repo="other", verbose=False)       # another model: its own key
    assert len(calls) == 3


def test_apply_small_m_allowlist_and_stale_cache(cal, monkeypatch):
    from dspark_rocm import small_m_qmm

    model = tiny_model("cpu", seed=2)
    keys = sorted({small_m_qmm.shape_key(m) for m in model.modules() if small_m_qmm.eligible(m)})
    calls = []
    monkeypatch.setattr(small_m_qmm, "measure_shapes", lambda *m, verbose=False: calls.append(1) or keys[:1])
    # a cache written under another key format: matches no module, so it is measured again
    cal.save_cached(f"{cal.device_key()}|smallm|t|None", ["4096x4096"])
    ids = cal.apply_small_m(model, target_repo="t", verbose=False)
    assert len(calls) == 1
    want = {id(m) for m in model.modules() if small_m_qmm.eligible(m) and small_m_qmm.shape_key(m) == keys[0]}
    assert ids == frozenset(want) and cal.SMALL_M_IDS == ids and ids
    assert cal.apply_small_m(model, target_repo="t", enabled=False, verbose=False) is None
    assert cal.SMALL_M_IDS is None


def test_attention_shape_probes(cal):
    from dspark_rocm.model import Target

    model = tiny_model("cpu", seed=3)
    a = model.args
    assert cal._attn_dims(model) == (a.num_attention_heads, a.num_key_value_heads, a.head_dim)

    class Wrapped:                                   # a Target-like object holding .model
        pass

    w = Wrapped()
    w.model = model
    assert cal._attn_dims(w) == cal._attn_dims(model)
    assert cal._attn_dims(object()) is None
    Target  # noqa: B018 - the real Target holds .model the same way

    class Attn:
        def __init__(self, **kw):
            self.n_heads, self.n_kv_heads, self.head_dim = 16, 8, 256
            self.__dict__.update(kw)

        def update_ctx(self):
            pass

    class Layer:
        def __init__(self, attn):
            self.self_attn = attn

    class Drafter:
        def __init__(self, attn):
            self.layers = [Layer(attn)]

    assert cal._drafter_attn_dims(Drafter(Attn())) == (16, 8, 256)
    assert cal._drafter_attn_dims(Drafter(Attn(sliding_window=2048))) is None
    assert cal._drafter_attn_dims(Drafter(Attn(causal_block=True))) is None
    assert cal._drafter_attn_dims(Drafter(Attn(sink=True))) is None
    assert cal._drafter_attn_dims(object()) is None


def test_apply_multirow_measures_target_and_drafter_shapes(cal, monkeypatch):
    from dspark_rocm import multirow_attn

    model = tiny_model("cpu", seed=4)
    seen = []

    def fake(hq, hk, d, verbose=False):
        seen.append((hq, hk, d))
        return ({"min_q": 2, "max_q": 8, "min_kv": 4096}, {}) if d == 128 else (None, {"reason": "no win"})

    monkeypatch.setattr(multirow_attn, "measure_window", fake)

    class Attn:
        n_heads, n_kv_heads, head_dim = 16, 8, 256

        def update_ctx(self):
            pass

    drafter = type("D", (), {"layers": [type("L", (), {"self_attn": Attn()})()]})()
    cfg = cal.apply_multirow_attn(model, drafter, verbose=False)
    a = model.args
    assert seen == [(a.num_attention_heads, a.num_key_value_heads, a.head_dim), (16, 8, 256)]
    assert cal.MULTIROW_CFG is cfg and len(cfg.windows) == 1
    w = cfg.window(a.num_attention_heads, a.num_key_value_heads, a.head_dim)
    assert (w.min_q, w.max_q, w.min_kv) == (2, 8, 4096)
    cal.apply_multirow_attn(model, drafter, verbose=False)             # cached: no new measurement
    assert len(seen) == 2
    assert cal.apply_multirow_attn(model, enabled=False) is None and cal.MULTIROW_CFG is None


def test_verify_scopes_install_in_the_reference_order(cal):
    from dspark_rocm import fast, multirow_attn, sdpa_split, small_m_qmm
    from dspark_rocm.nn import QuantizedLinear

    stock_sdpa, stock_fwd = fast.scaled_dot_product_attention, QuantizedLinear.forward
    with cal.verify_scopes():                                   # all off: nothing installed
        assert fast.scaled_dot_product_attention is stock_sdpa and QuantizedLinear.forward is stock_fwd
    cal.SDPA_SPLIT_CFG = sdpa_split.SplitConfig()
    cal.MULTIROW_CFG = multirow_attn.MultirowConfig((multirow_attn.Window(4, 2, 128),))
    cal.SMALL_M_IDS = frozenset({1})
    with cal.verify_scopes():
        assert multirow_attn.active() and small_m_qmm.active()
        # the multi-row patch sits over the split: what it does not serve falls to the split
        assert multirow_attn._fallthrough.value is sdpa_split._patched_call
        q = torch.randn(1, 4, 8, 16)
        k = torch.randn(1, 2, 64, 16)
        out = fast.scaled_dot_product_attention(q, k, k, scale=0.25, mask="causal")
        assert torch.allclose(out, fast.STOCK(q, k, k, scale=0.25, mask="causal"), atol=1e-5)
    assert fast.scaled_dot_product_attention is stock_sdpa and QuantizedLinear.forward is stock_fwd


def test_wide_gemm_threshold_measured_once_and_forced_threshold_verifies(cal, monkeypatch):
    from dspark_rocm import wide_gemm

    model = tiny_model("cpu", seed=5)
    calls = []

    def fake(*models):
        calls.append(len(models))
        return 512, ["k1"]

    monkeypatch.setattr(cal, "WIDE_GEMM_MIN_ROWS", None)
    monkeypatch.setattr(cal, "WIDE_GEMM_SHAPES", None)
    monkeypatch.setattr(wide_gemm, "measure_crossover", fake)
    assert cal.wide_gemm_min_rows(model, target_repo="t", verbose=False) == (512, ["k1"])
    assert cal.apply_wide_gemm(model, target_repo="t", verbose=False) == 512
    assert cal.WIDE_GEMM_SHAPES == ["k1"] and len(calls) == 1                # second call: cached
    monkeypatch.setattr(wide_gemm, "measure_crossover", lambda *m: None)
    assert cal.wide_gemm_min_rows(model, target_repo="u", verbose=False) == (None, [])
    seen = []
    monkeypatch.setattr(wide_gemm, "verified_shapes", lambda models, M, *a, **k: seen.append(M) or ["k2"])
    assert cal.apply_wide_gemm(model, target_repo="t", min_rows=64, verbose=False) == wide_gemm.SAFE_MIN_ROWS
    assert seen == [wide_gemm.SAFE_MIN_ROWS] and cal.WIDE_GEMM_SHAPES == ["k2"]  # verified at the clamped width
    assert cal.apply_wide_gemm(model, target_repo="t", min_rows=0, verbose=False) is None
    assert cal.WIDE_GEMM_SHAPES == []


def test_split_window_from_costs_kats(cal):
    """The window a stock-path cost sweep implies: widths whose balanced blocks cost together
    less than 95% of one call, the first consecutive run above the block size."""
    flat = {q: 1.0 for q in range(1, 17)}                         # cost independent of width: no gain
    assert cal.split_window_from_costs(flat, 4) is None
    linear = {q: float(q) for q in range(1, 17)}                  # cost per row constant: blocks never gain
    assert cal.split_window_from_costs(linear, 4) is None
    cliff = {q: (1.0 if q <= 5 else 6.0) for q in range(1, 17)}   # a cliff above 5 rows
    # 16 rows go as 4 blocks of 4 (4.0 against 6.0: a gain too)
    assert cal.split_window_from_costs(cliff, 5) == {"min_q": 6, "max_q": 16, "min_kv": 4096, "max_chunk": 5}
    # a width that does not gain ends the run
    gap = {**cliff, 9: 1.5}
    assert cal.split_window_from_costs(gap, 5) == {"min_q": 6, "max_q": 8, "min_kv": 4096, "max_chunk": 5}
    assert cal._split_chunk({1: 1.0, 2: 1.2, 4: 1.6, 8: 8.0}) == 4     # lowest cost per row up to 8 rows


def test_apply_sdpa_split_measures_once_and_obeys_enabled(cal, monkeypatch):
    from dspark_rocm import sdpa_split

    model = tiny_model("cpu", seed=6)
    calls = []

    def fake_costs(hq, hk, d, **kw):
        calls.append((hq, hk, d))
        return {q: (1.0 if q <= 4 else 5.0) for q in range(1, 17)}

    monkeypatch.setattr(cal, "_stock_attention_costs", fake_costs)
    cfg = cal.apply_sdpa_split(model, verbose=False)
    a = model.args
    assert calls == [(a.num_attention_heads, a.num_key_value_heads, a.head_dim)]
    assert cfg == sdpa_split.SplitConfig(min_q=5, max_q=16, min_kv=4096, max_chunk=4) and cal.SDPA_SPLIT_CFG is cfg
    assert cal.apply_sdpa_split(model, verbose=False) == cfg and len(calls) == 1      # cached
    assert cal.apply_sdpa_split(model, enabled=False) is None and cal.SDPA_SPLIT_CFG is None
    assert cal.apply_sdpa_split(model, enabled=True) == sdpa_split.SplitConfig()
    assert cal.apply_sdpa_split(object(), verbose=False) == sdpa_split.SplitConfig()  # shape unreadable
    monkeypatch.setattr(cal, "_stock_attention_costs", lambda *a, **k: {q: float(q) for q in range(1, 17)})
    assert cal.measure_split_window(8, 2, 64, refresh=True, verbose=False) is None
