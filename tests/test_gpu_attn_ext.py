"""GPU parity of verify attention at head dim 256, in fp16, and over quantized KV caches.

Bar: max|d| <= 2e-2 * RMS(out) against the float64 definition (oracle/attn_ref.py; the C
restatement for the 32k shape). Shapes follow the reference's serving range (D % 8 == 0,
D <= 256, bf16 or fp16: multirow_attn.py:200-214, :294-307): its headline 24/4/256 causal shape
at 32k (multirow_attn.py:25), the DSpark drafter's 16/8/256 non-causal context attention over a
4096-row window (config.py:166-169, model.py:199-242), tree masks, batch 2, strided cache views.

Quantized caches (mlx-lm QuantizedKVCache, 4- and 8-bit, groups of 64 along D: target.py:166-184)
are checked against dequantize-then-attend in float64, for being no less accurate than the plain
kernel over the same cache dequantized to bf16, and, on caches whose dequantized values are exact
in bf16 (power-of-two scales), within one output ulp of the plain kernel over those values: the
kernel's factored form (integer fields on the MFMA, scales and biases in fp32) computes the same
function, so any slip in its scale or bias handling shows there.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import assert_rms_close, rng
from oracle import attn_ref, c_oracle, quant_ref

pytestmark = pytest.mark.gpu

DT = {"bf16": torch.bfloat16, "f16": torch.float16}


def _round(a, dt):
    a = np.asarray(a, np.float32)
    return quant_ref.bf16_round(a) if dt == "bf16" else a.astype(np.float16).astype(np.float32)


def _mk(seed, B, hq, hk, mq, L, d, dt="bf16", slack=0):
    r = rng(seed)
    q = _round(r.standard_normal((B, hq, mq, d)), dt)
    k = _round(r.standard_normal((B, hk, L + slack, d)), dt)
    v = _round(r.standard_normal((B, hk, L + slack, d)), dt)
    return q, k, v


def _dev(a, dt, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev).to(DT[dt])


def _host(t):
    return t.float().cpu().numpy()


def _run(dev, q, k, v, L, scale, causal, dt="bf16", tree_anc=None):
    from dspark_rocm import ops

    anc = None if tree_anc is None else torch.tensor(np.asarray(tree_anc, dtype=np.int64), dtype=torch.int32)
    out = ops.verify_attention(_dev(q, dt, dev), _dev(k, dt, dev)[:, :, :L], _dev(v, dt, dev)[:, :, :L],
                               scale=scale, causal=causal, tree_anc=anc)
    assert out.dtype == DT[dt]
    return _host(out)


D256 = [
    # B, hq, hk, q_len, L, causal
    (1, 16, 8, 16, 4096, False),    # DSpark drafter context attention: 16 block rows, 4096-row window
    (1, 16, 8, 7, 4096, False),
    (1, 24, 4, 8, 1037, True),      # the reference's 24/4/256 shape, a short cache
    (1, 24, 4, 16, 3000, True),     # 96 rows: two row groups
    (2, 8, 8, 5, 129, True),        # MHA, batch 2
    (1, 4, 1, 3, 23, True),         # tail shorter than a tile
    (1, 32, 2, 4, 700, True),       # GQA 16
    (1, 32, 4, 16, 900, True),      # 128 rows: 6-tile workgroups, two row groups
    (1, 40, 4, 10, 640, True),      # 100 rows: one 6-tile workgroup, partly filled
]


@pytest.mark.parametrize("B,hq,hk,q_len,L,causal", D256)
def test_head_dim_256(dev, B, hq, hk, q_len, L, causal):
    q, k, v = _mk(hq * 7 + L, B, hq, hk, q_len, L, 256, slack=29)
    out = _run(dev, q, k, v, L, 256 ** -0.5, causal)
    ref = attn_ref.attention(q, k[:, :, :L], v[:, :, :L], 256 ** -0.5, causal=causal)
    assert_rms_close(out, ref, 2e-2, f"D=256 {hq}/{hk} q{q_len} L{L}")


def test_head_dim_256_headline_shape_32k(dev):
    """24 query / 4 KV heads x 256, 16 rows at a 32768-row offset (multirow_attn.py:25), causal."""
    Lt = 32768 + 16
    q, k, v = _mk(256, 1, 24, 4, 16, Lt, 256)
    out = _run(dev, q, k, v, Lt, 256 ** -0.5, True)
    ref = c_oracle.attention(quant_ref.bf16_bits(q), quant_ref.bf16_bits(k), quant_ref.bf16_bits(v), 256 ** -0.5, True)
    assert_rms_close(out, ref, 2e-2, "24/4/256 at 32k")


def test_head_dim_256_tree(dev):
    q, k, v = _mk(5, 1, 16, 4, 16, 900, 256)
    r = np.random.Generator(np.random.PCG64(3))
    anc = [1]
    for i in range(1, 16):
        anc.append(anc[int(r.integers(0, i))] | (1 << i))
    out = _run(dev, q, k, v, 900, 256 ** -0.5, False, tree_anc=anc)
    assert_rms_close(out, attn_ref.attention(q, k, v, 256 ** -0.5, tree_anc=anc), 2e-2, "D=256 tree")


ODD_D = [
    # d, B, hq, hk, q_len, L, causal: every head dim d % 8 == 0 up to 256 runs on the instance
    # above it (64, 128, 256) with the missing columns zero; strided views over a wider cache
    (8, 1, 8, 2, 5, 300, True),
    (40, 2, 8, 8, 3, 129, True),
    (72, 1, 32, 8, 16, 2064, True),      # 4-wave workgroups, split-KV blocks
    (96, 1, 64, 8, 16, 1500, True),      # 128 rows per KV head: 8-wave workgroups
    (112, 1, 32, 8, 16, 600, True),      # short cache: key-split workgroups
    (160, 1, 16, 8, 16, 1000, False),    # instance 256, non-causal
    (192, 1, 24, 4, 16, 3000, True),     # instance 256, 96 rows: 6-tile workgroups
    (248, 1, 4, 1, 3, 23, True),         # tail shorter than a tile
]


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("d,B,hq,hk,q_len,L,causal", ODD_D)
def test_any_head_dim_multiple_of_8(dev, dt, d, B, hq, hk, q_len, L, causal):
    q, k, v = _mk(d * 3 + L, B, hq, hk, q_len, L, d, dt=dt, slack=13)
    out = _run(dev, q, k, v, L, d ** -0.5, causal, dt=dt)
    ref = attn_ref.attention(q, k[:, :, :L], v[:, :, :L], d ** -0.5, causal=causal)
    assert_rms_close(out, ref, 2e-2, f"{dt} D={d} {hq}/{hk} q{q_len} L{L}")


def test_any_head_dim_tree_and_strided_out(dev):
    """Head dim 80 under a tree mask, written through the o-projection layout [B, Mq, Hq*D]:
    only the caller's 80 columns of each head are written (the bytes between stay untouched)."""
    from dspark_rocm import ops

    d, hq, hk, mq, L = 80, 16, 4, 12, 700
    q, k, v = _mk(80, 1, hq, hk, mq, L, d)
    r = np.random.Generator(np.random.PCG64(9))
    anc = [1]
    for i in range(1, mq):
        anc.append(anc[int(r.integers(0, i))] | (1 << i))
    ref = attn_ref.attention(q, k, v, d ** -0.5, tree_anc=anc)
    rows = torch.full((1, mq, hq * d + 8), 7.0, dtype=torch.bfloat16, device=dev)
    ops.verify_attention_into(_dev(q, "bf16", dev), _dev(k, "bf16", dev), _dev(v, "bf16", dev), rows,
                              (mq * (hq * d + 8), d, hq * d + 8), scale=d ** -0.5, causal=False,
                              tree_anc=torch.tensor(anc, dtype=torch.int32))
    got = _host(rows[:, :, :hq * d]).reshape(1, mq, hq, d).transpose(0, 2, 1, 3)
    assert_rms_close(got, ref, 2e-2, "D=80 tree, strided out")
    assert torch.all(rows[:, :, hq * d:] == 7.0)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("hq,hk,q_len,L,causal", [(32, 8, 16, 2064, True), (64, 8, 16, 4112, True),
                                                 (8, 2, 5, 300, False), (16, 8, 12, 1000, True)])
def test_fp16(dev, d, hq, hk, q_len, L, causal):
    q, k, v = _mk(d + hq + L, 1, hq, hk, q_len, L, d, dt="f16", slack=11)
    out = _run(dev, q, k, v, L, d ** -0.5, causal, dt="f16")
    ref = attn_ref.attention(q, k[:, :, :L], v[:, :, :L], d ** -0.5, causal=causal)
    assert_rms_close(out, ref, 2e-2, f"fp16 D={d} {hq}/{hk} q{q_len} L{L}")


# ---------------------------------------------------------------- quantized KV


def _quant_cache(seed, B, hk, L, d, bits, dt, slack):
    """A quantized cache holding L rows of N(0, 1) keys/values in a buffer of L + slack rows."""
    from dspark_rocm.quant import quantize_rows

    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    trips = []
    for _ in range(2):
        x = torch.randn((B, hk, L + slack, d), generator=g, device="cuda")
        w, s, b = quantize_rows(x, bits, 64, DT[dt])
        trips.append((w, s, b))
    views = [tuple(t[:, :, :L] for t in trip) for trip in trips]
    return views


def _host_trip(trip):
    w, s, b = trip
    return (w.cpu().numpy().view(np.uint32), s.float().cpu().numpy(), b.float().cpu().numpy())


def _dequant_on_device(trip, bits, dt):
    """scale * field + bias computed exactly (fp64), rounded to fp32 then to the compute type:
    the values of one fp32 fma followed by one rounding, as the kernel's loader forms them."""
    from dspark_rocm.quant import unpack

    w, s, b = trip
    lead = w.shape[:-1]
    f = unpack(w.reshape(-1, w.shape[-1]), bits).to(torch.float64).reshape(*lead, -1, 64)
    val = f * s.to(torch.float64).unsqueeze(-1) + b.to(torch.float64).unsqueeze(-1)
    return val.reshape(*lead, -1).to(torch.float32).to(DT[dt])


QCASES = [
    # B, hq, hk, q_len, L, d, causal
    (1, 32, 8, 16, 4112, 128, True),     # the 32/8/128 verify shape at 4k
    (1, 64, 8, 16, 2064, 128, True),     # 128 rows per KV head: 8-wave workgroups
    (1, 32, 8, 16, 600, 128, True),      # short cache: key-split workgroups
    (2, 8, 8, 5, 129, 64, True),         # batch 2, D 64
    (1, 16, 8, 16, 1500, 256, False),    # D 256, non-causal
    (1, 24, 4, 16, 1100, 256, True),     # D 256, 96 rows: the quantized path's 4-tile row groups
    (1, 4, 1, 3, 23, 64, True),          # tail shorter than a tile
]


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("B,hq,hk,q_len,L,d,causal", QCASES)
def test_quantized_kv(dev, bits, B, hq, hk, q_len, L, d, causal):
    from dspark_rocm import ops

    dt = "bf16"
    kq, vq = _quant_cache(L + d + bits, B, hk, L, d, bits, dt, slack=40)
    q = _mk(L + bits, B, hq, hk, q_len, 1, d)[0]
    qd = _dev(q, dt, dev)
    out = ops.verify_attention_quantized(qd, kq, vq, scale=d ** -0.5, causal=causal, bits=bits)
    ref = attn_ref.attention_quantized(q, _host_trip(kq), _host_trip(vq), d ** -0.5, bits, causal=causal)
    assert_rms_close(_host(out), ref, 2e-2, f"quantized {bits}-bit {hq}/{hk}x{d} q{q_len} L{L}")
    plain = ops.verify_attention(qd, _dequant_on_device(kq, bits, dt), _dequant_on_device(vq, bits, dt),
                                 scale=d ** -0.5, causal=causal)
    e_quant, e_plain = np.abs(_host(out) - ref).max(), np.abs(_host(plain) - ref).max()
    assert e_quant <= 1.05 * e_plain + 1e-6, (e_quant, e_plain)


def _exact_cache(seed, B, hk, L, d, bits, slack):
    """A quantized cache whose values scale * field + bias are exact in bf16: power-of-two
    scales and biases that are multiples of them."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    levels = (1 << bits) - 1
    trips = []
    for _ in range(2):
        f = torch.randint(0, levels + 1, (B * hk * (L + slack), d), generator=g, device="cuda")
        from dspark_rocm.quant import pack

        w = pack(f, bits).reshape(B, hk, L + slack, d * bits // 32)
        e = torch.randint(-6, -1, (B, hk, L + slack, d // 64), generator=g, device="cuda").float()
        sc = torch.exp2(e)
        bi = -sc * torch.randint(0, levels + 1, sc.shape, generator=g, device="cuda").float()
        trips.append((w, sc.to(torch.bfloat16), bi.to(torch.bfloat16)))
    return [tuple(t[:, :, :L] for t in trip) for trip in trips]


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("B,hq,hk,q_len,L,d,causal", [(1, 32, 8, 16, 2064, 128, True), (1, 64, 8, 16, 700, 128, True),
                                                      (1, 16, 8, 16, 1000, 256, False), (2, 8, 2, 5, 129, 64, True)])
def test_quantized_kv_factored_form_is_exact(dev, bits, B, hq, hk, q_len, L, d, causal):
    from dspark_rocm import ops

    kq, vq = _exact_cache(d + L + bits, B, hk, L, d, bits, slack=24)
    q = _mk(L + 3, B, hq, hk, q_len, 1, d)[0]
    qd = _dev(q, "bf16", dev)
    out = _host(ops.verify_attention_quantized(qd, kq, vq, scale=d ** -0.5, causal=causal, bits=bits))
    kd, vd = _dequant_on_device(kq, bits, "bf16"), _dequant_on_device(vq, bits, "bf16")
    assert torch.equal(kd.float(), _dequant_on_device(kq, bits, "f16").float())    # exact in both types
    plain = _host(ops.verify_attention(qd, kd, vd, scale=d ** -0.5, causal=causal))
    # both outputs are bf16 roundings of fp32 sums of the same exact terms: at most one ulp
    # apart (of the larger magnitude, so a rounding tie across a binade edge counts as one),
    # plus the fp32 scale of the factored form's two terms (each up to max|V|) for outputs
    # near zero, where they cancel
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.maximum(np.abs(plain), np.abs(out)), 1e-30))) - 7)
    floor = 1e-5 * float(np.abs(plain).max())
    assert np.all(np.abs(out - plain) <= ulp + floor), np.abs(out - plain).max()


@pytest.mark.parametrize("bits", [8, 4])
def test_quantized_kv_32k(dev, bits):
    """The 32/8/128 verify shape at a 32768-row offset over an 8- / 4-bit cache."""
    from dspark_rocm import ops

    Lt = 32768 + 16
    kq, vq = _quant_cache(bits, 1, 8, Lt, 128, bits, "bf16", slack=64)
    q = _mk(bits, 1, 32, 8, 16, 1, 128)[0]
    out = ops.verify_attention_quantized(_dev(q, "bf16", dev), kq, vq, scale=128 ** -0.5, causal=True, bits=bits)
    ref = attn_ref.attention_quantized(q, _host_trip(kq), _host_trip(vq), 128 ** -0.5, bits, causal=True)
    assert_rms_close(_host(out), ref, 2e-2, f"quantized {bits}-bit at 32k")


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("L", [2000, 32768 + 16])
def test_quantized_kv_fp16(dev, bits, L):
    """fp16 caches at 8 and 4 bits, up to the 32k verify shape: as accurate as the plain kernel
    over the dequantized cache (4-bit fields are unpacked exactly, no offset to cancel)."""
    from dspark_rocm import ops

    kq, vq = _quant_cache(77 + bits, 1, 8, L, 128, bits, "f16", slack=8)
    q = _mk(78 + bits, 1, 32, 8, 16, 1, 128, dt="f16")[0]
    qd = _dev(q, "f16", dev)
    out = ops.verify_attention_quantized(qd, kq, vq, scale=128 ** -0.5, causal=True, bits=bits)
    assert out.dtype == torch.float16
    ref = attn_ref.attention_quantized(q, _host_trip(kq), _host_trip(vq), 128 ** -0.5, bits, causal=True)
    assert_rms_close(_host(out), ref, 2e-2, f"quantized fp16 {bits}-bit L{L}")
    plain = ops.verify_attention(qd, _dequant_on_device(kq, bits, "f16"), _dequant_on_device(vq, bits, "f16"),
                                 scale=128 ** -0.5, causal=True)
    assert np.abs(_host(out) - ref).max() <= 1.05 * np.abs(_host(plain) - ref).max() + 1e-6


def test_quantized_cache_rollback_and_scope(dev):
    """QuantizedKVCache rows written, rolled back and rewritten: attention equals a fresh cache
    holding the committed rows; inside multirow_attention the quantized entry point runs the
    kernel (bitwise the direct call) and matches the stock dequantize path."""
    from dspark_rocm import fast, multirow_attn as mra, ops
    from dspark_rocm.kv_cache import QuantizedKVCache

    H, Hk, D, L0, mq = 32, 8, 128, 1200, 16
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    rand = lambda *s: torch.randn(s, generator=g, device=dev).to(torch.bfloat16)
    pre_k, pre_v, b1k, b1v, b2k, b2v = (rand(1, Hk, n, D) for n in (L0, L0, mq, mq, mq, mq))
    q2 = rand(1, H, mq, D)
    c = QuantizedKVCache(1, Hk, D, bits=8, device=dev, capacity=L0 + 64)
    c.update_and_fetch(pre_k, pre_v)
    c.update_and_fetch(b1k, b1v)
    c.trim(11)
    kk, vv = c.update_and_fetch(b2k, b2v)
    got = ops.verify_attention_quantized(q2, kk, vv, scale=D ** -0.5, causal=True, bits=8)
    f = QuantizedKVCache(1, Hk, D, bits=8, device=dev, capacity=L0 + 64)
    f.update_and_fetch(torch.cat([pre_k, b1k[:, :, :5]], dim=2), torch.cat([pre_v, b1v[:, :, :5]], dim=2))
    fk, fv = f.update_and_fetch(b2k, b2v)
    assert torch.equal(got, ops.verify_attention_quantized(q2, fk, fv, scale=D ** -0.5, causal=True, bits=8))
    cfg = mra.MultirowConfig((mra.Window(H, Hk, D, min_q=2, max_q=16, min_kv=64),))
    with mra.multirow_attention(cfg):
        routed = fast.quantized_scaled_dot_product_attention(q2, kk, vv, scale=D ** -0.5, mask="causal", bits=8)
        assert mra.why_not_quantized(q2, kk, vv, "causal", cfg, 64, 8) is None
    assert torch.equal(routed, got)
    stock = fast.quantized_scaled_dot_product_attention(q2, kk, vv, scale=D ** -0.5, mask="causal", bits=8)
    assert_rms_close(_host(got), _host(stock), 2e-2, "kernel vs stock quantized SDPA")


def test_refusals(dev):
    from dspark_rocm import _lib, ops

    for d in (100, 264):                                             # head_dim % 8 != 0, > 256
        q = torch.zeros((1, 8, 4, d), dtype=torch.bfloat16, device=dev)
        k = torch.zeros((1, 2, 64, d), dtype=torch.bfloat16, device=dev)
        with pytest.raises((_lib.DsparkError, ValueError)):
            ops.verify_attention(q, k, k, scale=0.1)
    q = torch.zeros((1, 8, 4, 64), dtype=torch.float16, device=dev)
    k = torch.zeros((1, 2, 64, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(TypeError):
        ops.verify_attention(q, k, k, scale=0.1)                     # mixed dtypes
    kq, vq = _quant_cache(1, 1, 2, 64, 64, 8, "bf16", slack=0)
    with pytest.raises(ValueError):
        ops.verify_attention_quantized(q.to(torch.bfloat16), kq, vq, scale=0.1, bits=4)   # words do not match bits
