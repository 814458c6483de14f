"""GPU parity of the multi-row verify attention (dspark_verify_attention) against the oracle.

Bar: max|Δ| <= 2e-2 * RMS(out) against the float64 definition; additionally within a few bf16
ulps of the restatement of the multirow kernel's arithmetic (bf16 P, fp32 partials). Cases
follow the reference's tests/test_multirow_attn.py:48-99 (GQA 1..16, off-grid KV lengths,
strided cache views, batch 2, row groups, causal and bidirectional, the causal leak KAT), plus
the tree mask, the 32/8-head verify shapes at L = 512..32k and KV rollback r in {0, 5, 15}.
"""

from __future__ import annotations

import numpy as np
import pytest

from _util import assert_rms_close, from_dev_bf16, max_abs, randn_bf16, rng, to_dev_bf16
from oracle import attn_ref, c_oracle, quant_ref

pytestmark = pytest.mark.gpu


def _mk(seed, B, hq, hk, mq, L, d, slack=0):
    r = rng(seed)
    q = randn_bf16(r, B, hq, mq, d)
    k = randn_bf16(r, B, hk, L + slack, d)
    v = randn_bf16(r, B, hk, L + slack, d)
    return q, k, v


def _gpu(dev, q, k, v, L, scale, causal, tree_anc=None):
    import torch

    from dspark_rocm import ops

    qd = to_dev_bf16(q, dev)
    kd = to_dev_bf16(k, dev)[:, :, :L, :]          # a KVCache-style view into a larger buffer
    vd = to_dev_bf16(v, dev)[:, :, :L, :]
    anc = None if tree_anc is None else torch.tensor(np.asarray(tree_anc, dtype=np.int64), dtype=torch.int32)
    return from_dev_bf16(ops.verify_attention(qd, kd, vd, scale=scale, causal=causal, tree_anc=anc))


CASES = [
    # B, hq, hk, q_len, L, d
    (1, 32, 8, 16, 528, 128),     # 32/8 heads, D 128 at L = 512 (+16 verify rows)
    (1, 32, 8, 15, 777, 128),     # DSpark drafter block, off-grid tail
    (1, 32, 8, 2, 64, 128),
    (1, 32, 2, 16, 500, 128),     # GQA 16 -> 256 rows: 4 row groups
    (2, 8, 8, 5, 129, 64),        # MHA, batch 2
    (1, 16, 2, 7, 16, 128),       # KV exactly the verify block
    (1, 4, 1, 3, 23, 64),         # MQA, tail shorter than a tile
    (1, 32, 8, 1, 300, 128),      # plain decode row
    (1, 24, 4, 8, 1037, 128),
    (1, 64, 8, 16, 4112, 128),    # the 64/8-head verify forward's shape: 128 rows, 2 row groups
]


@pytest.mark.parametrize("B,hq,hk,q_len,L,d", CASES)
@pytest.mark.parametrize("causal", [True, False])
def test_matches_reference(dev, B, hq, hk, q_len, L, d, causal):
    q, k, v = _mk(hash((B, hq, hk, q_len, L, d)) % 1000, B, hq, hk, q_len, L, d, slack=37)
    scale = d ** -0.5
    causal = causal and q_len > 1
    out = _gpu(dev, q, k, v, L, scale, causal)
    ref = attn_ref.attention(q, k[:, :, :L], v[:, :, :L], scale, causal=causal)
    assert_rms_close(out, ref, 2e-2, "vs fp64")
    # the kernel's own arithmetic class: within a few bf16 ulps of the restated multirow numerics
    mr = attn_ref.attention_multirow(q, k[:, :, :L], v[:, :, :L], scale, causal=causal)
    assert max_abs(out, ref) <= 2.0 * max_abs(mr, ref) + 4e-3, (max_abs(out, ref), max_abs(mr, ref))


def test_causal_rows_see_only_their_prefix(dev):
    """Leak KAT (tests/test_multirow_attn.py:90-99): masked keys dominate scores and values."""
    q, k, v = _mk(1, 1, 4, 4, 4, 64, 64)
    k[:, :, -3:] = 50.0
    v[:, :, -3:] = 1e3
    out = _gpu(dev, q, k, v, 64, 0.125, True)
    ref = attn_ref.attention(q, k, v, 0.125, causal=True)
    assert max_abs(out, ref) < 50.0
    # row 0 must not see any of the last 3 keys: its output stays O(1)
    assert np.max(np.abs(out[:, :, 0])) < 10.0


def test_tree_mask(dev):
    mq, L = 8, 300
    q, k, v = _mk(2, 1, 16, 4, mq, L, 128)
    anc = [1, 3, 5, 9, 17, 49, 0b1100001, 0b10100001]   # ancestor-or-self bits per row
    out = _gpu(dev, q, k, v, L, 128 ** -0.5, False, tree_anc=anc)
    ref = attn_ref.attention(q, k, v, 128 ** -0.5, tree_anc=anc)
    assert_rms_close(out, ref, 2e-2, "tree")


def _tree16(seed):
    """Ancestor-or-self bits for a 16-row draft tree: row i's parent is a random earlier row."""
    r = np.random.Generator(np.random.PCG64(seed))
    anc = [1]
    for i in range(1, 16):
        anc.append(anc[int(r.integers(0, i))] | (1 << i))
    return anc


@pytest.mark.parametrize("hq,hk,L,d", [
    (64, 8, 4112, 128),    # 128 rows per KV head: 8-wave workgroups, two tiles in flight
    (64, 8, 1000, 64),     # same at head_dim 64, a short cache
    (32, 8, 16400, 128),   # 64 rows, long cache: 4-wave workgroups
    (32, 8, 600, 128),     # 64 rows, short cache: 8 waves splitting each tile's keys
])
def test_tree_mask_every_workgroup_shape(dev, hq, hk, L, d):
    q, k, v = _mk(hq + L + d, 1, hq, hk, 16, L, d)
    anc = _tree16(L)
    out = _gpu(dev, q, k, v, L, d ** -0.5, False, tree_anc=anc)
    ref = attn_ref.attention(q, k, v, d ** -0.5, tree_anc=anc)
    assert_rms_close(out, ref, 2e-2, f"tree hq={hq} L={L} d={d}")


@pytest.mark.parametrize("L", [512, 4096, 16384, 32768])
def test_32x8x128_cache_lengths(dev, L):
    """32 q heads, 8 KV heads, D 128, 16 rows at offset L (L + 16 keys), split-KV."""
    from dspark_rocm import ops

    Lt = L + 16
    q, k, v = _mk(L, 1, 32, 8, 16, Lt, 128)
    out = _gpu(dev, q, k, v, Lt, 128 ** -0.5, True)
    ref = c_oracle.attention(quant_ref.bf16_bits(q), quant_ref.bf16_bits(k), quant_ref.bf16_bits(v), 128 ** -0.5, True)
    assert_rms_close(out, ref, 2e-2, f"verify attention L={L}")
    assert ops.verify_attention_blocks(1, 32, 8, 16, 128, Lt) >= 1


@pytest.mark.parametrize("r", [0, 5, 15])
def test_rollback_then_rewrite(dev, r):
    """Verify 16 rows at offset L0, reject r, write a new 16-row block at the trimmed offset:
    identical to a fresh cache holding only the committed prefix (target.py:679-696,
    batch_engine.py:220-224 — trim is metadata, the next write overwrites)."""
    import torch

    from dspark_rocm import ops
    from dspark_rocm.kv_cache import KVCache

    H, Hk, D, L0, mq = 32, 8, 128, 1000, 16
    rg = rng(40 + r)
    prefix_k, prefix_v = randn_bf16(rg, 1, Hk, L0, D), randn_bf16(rg, 1, Hk, L0, D)
    blk1_k, blk1_v = randn_bf16(rg, 1, Hk, mq, D), randn_bf16(rg, 1, Hk, mq, D)
    blk2_k, blk2_v = randn_bf16(rg, 1, Hk, mq, D), randn_bf16(rg, 1, Hk, mq, D)
    q1, q2 = randn_bf16(rg, 1, H, mq, D), randn_bf16(rg, 1, H, mq, D)
    c = KVCache(1, Hk, D, device=dev, capacity=L0 + 64)
    c.update_and_fetch(to_dev_bf16(prefix_k, dev), to_dev_bf16(prefix_v, dev))
    kk, vv = c.update_and_fetch(to_dev_bf16(blk1_k, dev), to_dev_bf16(blk1_v, dev))
    ops.verify_attention(to_dev_bf16(q1, dev), kk, vv, scale=D ** -0.5, causal=True)
    c.trim(r)
    assert c.offset == L0 + mq - r
    kk, vv = c.update_and_fetch(to_dev_bf16(blk2_k, dev), to_dev_bf16(blk2_v, dev))
    got = from_dev_bf16(ops.verify_attention(to_dev_bf16(q2, dev), kk, vv, scale=D ** -0.5, causal=True))
    keep = mq - r
    fk = np.concatenate([prefix_k, blk1_k[:, :, :keep], blk2_k], axis=2)
    fv = np.concatenate([prefix_v, blk1_v[:, :, :keep], blk2_v], axis=2)
    fresh = _gpu(dev, q2, fk, fv, fk.shape[2], D ** -0.5, True)
    assert np.array_equal(got, fresh)
    ref = attn_ref.attention(q2, fk, fv, D ** -0.5, causal=True)
    assert_rms_close(got, ref, 2e-2, f"rollback r={r}")


def test_rows_independent_of_block(dev):
    """Row i of a 16-row verify equals a 1-row call over keys 0..L-16+i (sdpa_split.py:9-14)."""
    mq, L = 16, 2064
    q, k, v = _mk(6, 1, 32, 8, mq, L, 128)
    full = _gpu(dev, q, k, v, L, 128 ** -0.5, True)
    for i in (0, 7, 15):
        Li = L - mq + i + 1
        one = _gpu(dev, q[:, :, i:i + 1], k[:, :, :Li], v[:, :, :Li], Li, 128 ** -0.5, True)
        assert_rms_close(full[:, :, i:i + 1], one, 2e-2, f"row {i}")


def test_refusals(dev):
    import torch

    from dspark_rocm import _lib, ops

    q = torch.zeros((1, 8, 4, 100), dtype=torch.bfloat16, device=dev)
    k = torch.zeros((1, 2, 64, 100), dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.DsparkError):
        ops.verify_attention(q, k, k, scale=0.1)          # head_dim 100: not a multiple of 8
    q = torch.zeros((1, 6, 4, 64), dtype=torch.bfloat16, device=dev)
    k = torch.zeros((1, 4, 64, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.DsparkError):
        ops.verify_attention(q, k, k, scale=0.1)          # Hq % Hk != 0
