"""GPU: the 32B-class dense 8-bit verify step (hidden 5120, 64/8 heads x 128, intermediate
25600, vocabulary 151936, RoPE 1e6) at its real size, 16 verify rows over a 16384-row cache.

- one full-width layer plus the final norm, the 151936-row lm_head and the device argmax, op
  by op on the engine's own buffers: each kernel against the oracle applied to that kernel's
  actual inputs (projections and attention within 2e-2 x RMS, the elementwise kernels at their
  unit tests' bars, argmax exact), then the whole step (``Target.verify``) bitwise equal to the
  staged ops and within 5e-2 x RMS of the chained oracle forward, with greedy tokens equal
  wherever the oracle's top-2 margin exceeds twice the error (target.py:642-677,
  generate.py:1544-1593);
- all 64 layers: the step reading the packed weight form is bitwise the step reading the
  reference layout, and verify -> rollback(11) -> verify is bitwise independent of what the
  rolled-back rows held (target.py:679-696).

The oracle's wide projections go through its C restatement (model_ref.qmm_c).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _model_util import to_ref
from _util import assert_rms_close
from oracle import attn_ref, c_oracle, model_ref, moe_ref, quant_ref

pytestmark = pytest.mark.gpu

DENSE_5120 = dict(hidden_size=5120, intermediate_size=25600, num_attention_heads=64, num_key_value_heads=8, head_dim=128,
          vocab_size=151936, rms_norm_eps=1e-6, rope_theta=1e6, bits=8, lm_head_bits=8)
CTX, ROWS = 16384, 16


def _np(t):
    return t.detach().float().cpu().numpy()


def _model(dev, layers, seed):
    from dspark_rocm.model import DenseModel, ModelArgs

    return DenseModel.random(ModelArgs(num_hidden_layers=layers, **DENSE_5120), device=dev, seed=seed)


def _seed_prefix(caches, seed):
    """The synthetic 16k prefix (random bf16 K/V rows, as calibrate.py:214-244 inflates a cache)."""
    g = torch.Generator(device=caches[0].keys.device)
    g.manual_seed(seed)
    for c in caches:
        c.keys[:, :, :CTX].normal_(generator=g)
        c.values[:, :, :CTX].normal_(generator=g)
        c.offset = CTX


class _Rows:
    """Embedding rows fetched from the device table on demand (no 3 GB host copy)."""

    def __init__(self, table):
        self.table = table

    def __getitem__(self, ids):
        return _np(self.table[torch.as_tensor(np.asarray(ids), device=self.table.device)])


def _ulps_close(got, want, what, ulps=2):
    """Elementwise within ``ulps`` bf16 ulps of the oracle (plus a floor near zero)."""
    tol = ulps * 2.0 ** -8 * np.abs(want) + 1e-3 * float(np.sqrt(np.mean(np.square(want, dtype=np.float64))))
    bad = np.abs(got - want) > tol
    assert not bad.any(), f"{what}: {bad.sum()} elements beyond {ulps} ulps, worst {np.abs(got - want).max():.4g}"


def test_dense_5120_layer_and_head_full_width_against_oracle(dev):
    from dspark_rocm import ops
    from dspark_rocm.model import Target

    model = _model(dev, 1, seed=51)
    a = model.args
    H, hq, hk, d, eps = a.hidden_size, a.num_attention_heads, a.num_key_value_heads, a.head_dim, a.rms_norm_eps
    tgt = Target(model)
    e = tgt.engine
    layer = model.layers[0]
    at, mlp = layer.self_attn, layer.mlp
    assert id(mlp) in e._swiglu and id(at.q_proj) in e._packed and id(model.lm_head) in e._packed
    cache = tgt.make_cache(CTX + 64)
    _seed_prefix(cache, 52)
    ref = to_ref(model, matmul=model_ref.qmm_c, embed=_Rows(model.embed_tokens))
    lay = ref.layers[0]
    ids = np.random.Generator(np.random.PCG64(53)).integers(0, a.vocab_size, ROWS)
    M, L = ROWS, CTX + ROWS
    c = cache[0]

    # ---- staged: every kernel of the step on the engine's buffers, checked on its own inputs
    c.reserve(M)
    e.ids[:M].copy_(torch.as_tensor(ids, device=dev))
    h, r, y = e.h[:M], e.r[:M], e.y[:M]
    torch.index_select(model.embed_tokens, 0, e.ids[:M], out=h)
    ops.rmsnorm(h, layer.input_layernorm, eps, out=y)
    y0 = _np(y)
    assert np.abs(y0 - model_ref.rmsnorm(_np(h), lay["input_norm"], eps)).max() <= 2 ** -7 * np.abs(y0).max()
    e._qmm(y, [at.q_proj, at.k_proj, at.v_proj], [e.q[:M], e.k[:M], e.v[:M]])
    for name, buf in (("q", e.q), ("k", e.k), ("v", e.v)):
        want = model_ref.qmm_c(y0, lay[name])
        assert_rms_close(_np(buf[:M]), want, 2e-2, f"{name}_proj")
        _ulps_close(_np(buf[:M]), want, f"{name}_proj")
    qatt = e.qatt[:, :, :M]
    ops.qk_norm_rope_kv(e.q[:M], e.k[:M], e.v[:M], at.q_norm, at.k_norm, heads=hq, kv_heads=hk, head_dim=d, eps=eps,
                        rope_base=a.rope_theta, pos0=CTX, q_out=qatt[0], k_cache=c.keys[0], v_cache=c.values[0])
    pos = np.arange(CTX, CTX + M)
    q_ref = model_ref.rope(model_ref.rmsnorm(_np(e.q[:M]).reshape(M, hq, d).transpose(1, 0, 2), lay["q_norm"], eps),
                           pos, a.rope_theta)
    k_ref = model_ref.rope(model_ref.rmsnorm(_np(e.k[:M]).reshape(M, hk, d).transpose(1, 0, 2), lay["k_norm"], eps),
                           pos, a.rope_theta)
    tol = 2 ** -6 * max(np.abs(q_ref).max(), 1.0)
    assert np.abs(_np(qatt[0]) - q_ref).max() <= tol
    assert np.abs(_np(c.keys[0, :, CTX:L]) - k_ref).max() <= tol
    assert np.array_equal(_np(c.values[0, :, CTX:L]), _np(e.v[:M]).reshape(M, hk, d).transpose(1, 0, 2))
    kv, vv = c.keys[:, :, :L], c.values[:, :, :L]
    att = e.att[:M]
    ops.verify_attention_into(qatt, kv, vv, att, (M * hq * d, d, hq * d), scale=d ** -0.5, causal=True,
                              workspace=e.attn_ws)
    kb = quant_ref.bf16_bits(_np(kv))
    vb = quant_ref.bf16_bits(_np(vv))
    att_ref = c_oracle.attention(quant_ref.bf16_bits(_np(qatt)), kb, vb, d ** -0.5, causal=True)
    att_ref = model_ref.bf(att_ref[0].transpose(1, 0, 2).reshape(M, hq * d))
    assert_rms_close(_np(att), att_ref, 2e-2, "attention (64/8 heads, 16 rows over 16400 keys)")
    exact = attn_ref.attention(_np(qatt)[:, :8], _np(kv)[:, :1], _np(vv)[:, :1], d ** -0.5, causal=True)
    assert_rms_close(_np(att).reshape(M, hq, d)[:, :8].transpose(1, 0, 2), exact[0], 2e-2,
                     "attention, KV head 0, float64 definition")
    e._qmm(att, [at.o_proj], [r])
    assert_rms_close(_np(r), model_ref.qmm_c(_np(att), lay["o"]), 2e-2, "o_proj")
    h_before = _np(h)
    ops.rmsnorm(h, layer.post_attention_layernorm, eps, residual=r, h_out=h, out=y)
    assert np.array_equal(_np(h), model_ref.bf(h_before + _np(r)))
    y1 = _np(y)
    assert np.abs(y1 - model_ref.rmsnorm(_np(h), lay["post_norm"], eps)).max() <= 2 ** -7 * np.abs(y1).max()
    ops.quantized_swiglu_packed(y, e._swiglu[id(mlp)], out=e.hm[:M], workspace=e.qmm_ws)
    # the gate and up projections at the projection bar (unfused launch, reference layout) ...
    g_un, u_un = ops.quantized_matmul_multi([y], [mlp.gate_proj.weight, mlp.up_proj.weight],
                                            [mlp.gate_proj.scales, mlp.up_proj.scales],
                                            [mlp.gate_proj.biases, mlp.up_proj.biases], bits=a.bits)
    g_ref, u_ref = model_ref.qmm_c(y1, lay["gate"]), model_ref.qmm_c(y1, lay["up"])
    for name, got_p, want_p in (("gate_proj", g_un, g_ref), ("up_proj", u_un, u_ref)):
        assert_rms_close(_np(got_p), want_p, 2e-2, name)
        _ulps_close(_np(got_p), want_p, name)
    # ... the fused launch bitwise the unfused one plus SwiGLU, which is exactly the oracle's
    # SwiGLU formula on those inputs, and the result within the ulps two rounded inputs allow
    assert np.array_equal(_np(e.hm[:M]), moe_ref.swiglu(_np(g_un), _np(u_un)))
    assert torch.equal(e.hm[:M], ops.swiglu(g_un, u_un))
    _ulps_close(_np(e.hm[:M]), moe_ref.swiglu(g_ref, u_ref), "fused gate/up/SwiGLU (I = 25600)", ulps=4)
    e._qmm(e.hm[:M], [mlp.down_proj], [r])
    assert_rms_close(_np(r), model_ref.qmm_c(_np(e.hm[:M]), lay["down"]), 2e-2, "down_proj (K = 25600)")
    h_before = _np(h)
    ops.rmsnorm(h, model.norm, eps, residual=r, h_out=h, out=y)
    assert np.array_equal(_np(h), model_ref.bf(h_before + _np(r)))
    y2 = _np(y)
    assert np.abs(y2 - model_ref.rmsnorm(_np(h), ref.norm, eps)).max() <= 2 ** -7 * np.abs(y2).max()
    logits = e.logits[:M]
    e._qmm(y, [model.lm_head], [logits])
    staged = logits.clone()
    lm_ref = model_ref.qmm_c(y2, ref.lm_head)
    assert_rms_close(_np(staged), lm_ref, 2e-2, "lm_head (151936 x 5120)")
    _ulps_close(_np(staged), lm_ref, "lm_head")
    tt = ops.argmax_rows(staged)
    assert tt.cpu().tolist() == [int(i) for i in _np(staged).argmax(-1)]

    # ---- the whole step (fresh cache, same prefix): bitwise the staged ops, and the chained
    # oracle forward within the end-to-end bar
    cache2 = tgt.make_cache(CTX + 64)
    _seed_prefix(cache2, 52)
    got, _ = tgt.verify(torch.as_tensor(ids[None]), cache2)
    assert torch.equal(got[0], staged)
    assert torch.equal(cache2[0].keys[:, :, :L], c.keys[:, :, :L])
    ref.seed_cache([_np(cache2[0].keys[0, :, :CTX])], [_np(cache2[0].values[0, :, :CTX])])
    want = ref.forward(ids.tolist())
    err, _ = assert_rms_close(_np(got[0]), want, 5e-2, "verify step (1 layer + head) vs chained oracle")
    top2 = np.sort(want, axis=-1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * err
    assert clear.sum() >= M // 2, "too few rows with a clear greedy token to check"
    assert np.array_equal(_np(got[0]).argmax(-1)[clear], want.argmax(-1)[clear])


def test_dense_5120_64_layers_packed_is_reference_layout_and_rollback_is_exact(dev):
    from dspark_rocm.model import Target

    model = _model(dev, 64, seed=61)
    a = model.args
    packed, plain = Target(model, packed=True), Target(model, packed=False)
    assert len(packed.engine._swiglu) == 64 and not plain.engine._packed
    caches = [packed.make_cache(CTX + 64), plain.make_cache(CTX + 64), packed.make_cache(CTX + 64)]
    _seed_prefix(caches[0], 62)
    for c in caches[1:]:
        for src, dst in zip(caches[0], c):
            dst.keys.copy_(src.keys)
            dst.values.copy_(src.values)
            dst.offset = src.offset
    r = np.random.Generator(np.random.PCG64(63))
    block1 = r.integers(0, a.vocab_size, ROWS)
    block2 = r.integers(0, a.vocab_size, ROWS)
    stale = block1.copy()
    stale[5:] = r.integers(0, a.vocab_size, ROWS - 5)          # rows rolled back below: must not matter
    outs = []
    for tgt, cache, first in ((packed, caches[0], block1), (plain, caches[1], block1), (packed, caches[2], stale)):
        l1, _ = tgt.verify(torch.as_tensor(first[None]), cache)
        tgt.rollback(cache, ROWS - 5)
        assert cache[0].offset == CTX + 5 and cache[-1].offset == CTX + 5
        l2, _ = tgt.verify(torch.as_tensor(block2[None]), cache)
        outs.append((l1.clone(), l2.clone()))
        torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]), "first verify: packed vs reference layout"
    assert torch.equal(outs[0][1], outs[1][1]), "verify after rollback: packed vs reference layout"
    assert torch.equal(outs[0][0][0, :5], outs[2][0][0, :5]), "rows before the differing drafts"
    assert torch.equal(outs[0][1], outs[2][1]), "verify after rollback depends on rolled-back rows"
    assert torch.isfinite(outs[0][1].float()).all()
