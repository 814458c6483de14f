"""GPU: the dense verify forward over the reference's wider serving range.

- quantized KV caches (mlx-lm QuantizedKVCache, every layer's cache when the target has
  kv_bits, target.py:166-184): the cache-writing kernel quantizes exactly the rows the plain
  kernel writes, by the build quantizer's rule (bitwise); the fused step over 8- and 4-bit
  caches against the oracle forward with quantized caches, over verify blocks with rollback; the
  module path over the same caches against the fused step; one full-width 32B-class layer
  (hidden 5120, 64/8 x 128, intermediate 25600) plus head over an 8-bit cache at 16k;
- head dim 256 (the reference's measured 24/4/256 target family, multirow_attn.py:25): the
  fused step for a 24/4/256 model against the oracle forward with rollback.

Bars: each kernel's own (bitwise for the cache write); the whole multi-layer forward within
5e-2 x RMS of the oracle, greedy tokens equal wherever the oracle's top-2 margin exceeds twice
the error.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _model_util import tiny_model, to_ref
from _util import assert_rms_close

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _check_forward(got, want, what):
    err, _ = assert_rms_close(_np(got), want, 5e-2, what)
    top2 = np.sort(want, axis=-1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * err
    assert np.array_equal(_np(got).argmax(-1)[clear], want.argmax(-1)[clear]), what


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("D,Hq,Hk", [(64, 8, 2), (128, 8, 2), (256, 6, 3)])
def test_quantized_cache_write_is_the_quantizer_on_the_plain_rows(dev, bits, D, Hq, Hk):
    from dspark_rocm import ops
    from dspark_rocm.quant import quantize_rows

    M, pos0, cap = 16, 3000, 3000 + 40
    g = torch.Generator(device=dev)
    g.manual_seed(D + bits)
    q = torch.randn((M, Hq * D), generator=g, device=dev).to(torch.bfloat16)
    k = (3 * torch.randn((M, Hk * D), generator=g, device=dev)).to(torch.bfloat16)
    v = torch.randn((M, Hk * D), generator=g, device=dev).to(torch.bfloat16)
    v[3, :64] = 0.5                                                   # a flat group: scale 0
    qw = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kc = torch.zeros((Hk, cap, D), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    qo = torch.empty((Hq, M, D), dtype=torch.bfloat16, device=dev)
    kwargs = dict(heads=Hq, kv_heads=Hk, head_dim=D, eps=1e-6, rope_base=1e6, pos0=pos0)
    ops.qk_norm_rope_kv(q, k, v, qw, kw, q_out=qo, k_cache=kc, v_cache=vc, **kwargs)

    def trip():
        W, G = D * bits // 32, D // 64
        return (torch.full((Hk, cap, W), -1, dtype=torch.int32, device=dev),
                torch.full((Hk, cap, G), 7.0, dtype=torch.bfloat16, device=dev),
                torch.full((Hk, cap, G), 7.0, dtype=torch.bfloat16, device=dev))

    kq, vq = trip(), trip()
    qo2 = torch.empty_like(qo)
    ops.qk_norm_rope_kv_quantized(q, k, v, qw, kw, q_out=qo2, k_cache=kq, v_cache=vq, bits=bits, **kwargs)
    assert torch.equal(qo2, qo)
    rows = slice(pos0, pos0 + M)
    for (w, s, b), plain in ((kq, kc), (vq, vc)):
        ww, ss, bb = quantize_rows(plain[:, rows], bits, 64, torch.bfloat16)
        assert torch.equal(w[:, rows], ww) and torch.equal(s[:, rows], ss) and torch.equal(b[:, rows], bb)
        assert (w[:, :pos0] == -1).all() and (w[:, pos0 + M:] == -1).all()      # nothing outside the rows
        assert (s[:, :pos0] == 7).all() and (b[:, pos0 + M:] == 7).all()
    assert (vq[1][0, pos0 + 3, 0] == 0).item()                                  # the flat group's scale


@pytest.mark.parametrize("bits", [8, 4])
def test_verify_over_quantized_caches_matches_oracle_with_rollback(dev, bits):
    from dspark_rocm.model import Target

    model = tiny_model(dev, seed=20 + bits)
    ref = to_ref(model, kv_bits=bits)
    tgt = Target(model, kv_bits=bits)
    cache = tgt.make_cache(128)
    assert all(c.bits == bits for c in cache)
    r = np.random.Generator(np.random.PCG64(bits))
    for n, rej in ((16, 0), (9, 5), (16, 15), (1, 0), (12, 3)):
        ids = r.integers(0, 512, n).tolist()
        got, _ = tgt.verify(torch.tensor([ids]), cache)
        _check_forward(got[0], ref.forward(ids), f"{bits}-bit KV verify block of {n}")
        tgt.rollback(cache, rej)
        ref.trim(rej)
        assert cache[0].offset == ref.offset


@pytest.mark.parametrize("bits", [8, 4])
def test_module_path_over_quantized_caches_matches_fused(dev, bits):
    """The module path routes a quantized cache to quantized_scaled_dot_product_attention
    (mlx-lm's per-cache dispatch); its caches hold exactly what the fused step's kernel wrote."""
    from dspark_rocm.model import Target

    model = tiny_model(dev, seed=30 + bits)
    tgt = Target(model, kv_bits=bits)
    ca, cb = tgt.make_cache(64), tgt.make_cache(64)
    ids = torch.tensor([[3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5, 8, 9, 7]])
    fused, _ = tgt.verify(ids, ca)
    with torch.no_grad():
        mod = model(ids.to(dev), cb)
    assert_rms_close(_np(mod[0]), _np(fused[0]), 5e-2, "module path vs fused over quantized caches")
    # the first layer's cache rows: the module path quantizes the same rotated k (torch ops for
    # norm and RoPE, which round like the kernel) -- equal fields where the values agree
    wa, wb = ca[0].keys[0][:, :, :14], cb[0].keys[0][:, :, :14]
    assert (wa == wb).float().mean().item() > 0.95


def test_dense_5120_layer_over_8bit_kv_cache_against_oracle(dev):
    """One full-width 32B-class layer (hidden 5120, 64/8 heads x 128, intermediate 25600,
    vocabulary 151936) over a 16k 8-bit quantized cache: 16 verify rows through the fused step
    against the oracle forward over the same dequantized prefix with quantized new rows."""
    from dspark_rocm.model import DenseModel, ModelArgs, Target
    from dspark_rocm.quant import quantize_rows

    from test_gpu_dense_verify_full import DENSE_5120, CTX, ROWS, _Rows
    from oracle import model_ref, quant_ref

    model = DenseModel.random(ModelArgs(num_hidden_layers=1, **DENSE_5120), device=dev, seed=71)
    a = model.args
    tgt = Target(model, kv_bits=8)
    cache = tgt.make_cache(CTX + 64)
    g = torch.Generator(device=dev)
    g.manual_seed(72)
    c = cache[0]
    for trip in (c.keys, c.values):
        x = torch.randn((1, a.num_key_value_heads, CTX, a.head_dim), generator=g, device=dev).to(torch.bfloat16)
        for buf, part in zip(trip, quantize_rows(x, 8, 64, torch.bfloat16)):
            buf[:, :, :CTX] = part
    c.offset = CTX
    ref = to_ref(model, matmul=model_ref.qmm_c, embed=_Rows(model.embed_tokens), kv_bits=8)

    def deq(trip):
        w, s, b = (t[0, :, :CTX] for t in trip)
        hk, L, W = w.shape
        vals = quant_ref.dequantize(w.reshape(hk * L, W).cpu().numpy().view(np.uint32),
                                    _np(s).reshape(hk * L, -1), _np(b).reshape(hk * L, -1), 8)
        return vals.reshape(hk, L, -1)

    ref.seed_cache([deq(c.keys)], [deq(c.values)])
    ids = np.random.Generator(np.random.PCG64(73)).integers(0, a.vocab_size, ROWS)
    got, _ = tgt.verify(torch.as_tensor(ids[None]), cache)
    want = ref.forward(ids.tolist())
    err, _ = assert_rms_close(_np(got[0]), want, 5e-2, "5120-hidden layer + head over an 8-bit KV cache at 16k")
    top2 = np.sort(want, axis=-1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 2 * err
    assert clear.sum() >= ROWS // 2
    assert np.array_equal(_np(got[0]).argmax(-1)[clear], want.argmax(-1)[clear])


def test_head_dim_256_target_matches_oracle_with_rollback(dev):
    """A 24/4-head x 256 target (the reference's Qwen3.8-27B attention shape class) through the
    fused step: q/k norm + RoPE at head dim 256, 96 rows per KV head in the attention kernel."""
    from dspark_rocm.model import Target

    model = tiny_model(dev, seed=40, hidden_size=1024, intermediate_size=2048, num_attention_heads=24,
                       num_key_value_heads=4, head_dim=256)
    ref = to_ref(model)
    tgt = Target(model)
    cache = tgt.make_cache(256)
    r = np.random.Generator(np.random.PCG64(41))
    for n, rej in ((16, 3), (16, 0), (5, 4), (16, 15), (8, 0)):
        ids = r.integers(0, 512, n).tolist()
        got, _ = tgt.verify(torch.tensor([ids]), cache)
        _check_forward(got[0], ref.forward(ids), f"24/4/256 verify block of {n}")
        tgt.rollback(cache, rej)
        ref.trim(rej)
