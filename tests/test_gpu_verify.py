"""GPU: the dense verify forward (the 64-layer verify step's path) against the oracle.

- layer kernels (residual + RMSNorm, q/k norm + RoPE + cache write, SwiGLU, argmax, greedy
  accept) against oracle/model_ref.py, moe_ref.swiglu and verify_ref (bit-exact for indices);
- Target.verify (fused engine) logits against the numpy forward of the same weights over
  several verify blocks with rollback (max|d| <= 5e-2 * RMS for the whole two-layer forward,
  greedy tokens equal wherever the top-2 margin exceeds the error); the module path under the
  reference's scopes against the fused engine;
- the fixed-seed synthetic speculative trace: tokens committed by greedy speculative rounds
  equal plain greedy decoding, and the mean accepted length equals the one the draft's
  corruption pattern implies (generate.py:1544-1593, :111-113).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _model_util import tiny_model, to_ref
from _util import ROPE_KAT_TOL, assert_rms_close, rope_kat_errors
from oracle import model_ref, moe_ref, verify_ref

pytestmark = pytest.mark.gpu


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("H", [5120, 8192, 8200, 16384])   # rows held in registers up to 8192
def test_rmsnorm_kernel(dev, H):
    from dspark_rocm import ops

    g = torch.Generator(device=dev)
    g.manual_seed(H)
    x = torch.randn((16, H), generator=g, device=dev).to(torch.bfloat16)
    r = torch.randn((16, H), generator=g, device=dev).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
    y = ops.rmsnorm(x, w, 1e-6)
    assert np.array_equal(_np(y), model_ref.rmsnorm(_np(x), _np(w), 1e-6)) or \
        np.abs(_np(y) - model_ref.rmsnorm(_np(x), _np(w), 1e-6)).max() <= 2 ** -7 * np.abs(_np(y)).max()
    h_ref = model_ref.bf(_np(x) + _np(r))
    hh = x.clone()
    y2 = ops.rmsnorm(hh, w, 1e-6, residual=r, h_out=hh)              # in place, as the engine runs it
    assert np.array_equal(_np(hh), h_ref)
    assert np.abs(_np(y2) - model_ref.rmsnorm(h_ref, _np(w), 1e-6)).max() <= 2 ** -7 * np.abs(h_ref).max()


@pytest.mark.parametrize("D", [64, 96, 128, 256])
@pytest.mark.parametrize("Hq,Hk", [(8, 2), (5, 1)])   # 5 + 2 heads: a partly filled workgroup
def test_qk_norm_rope_kv_kernel(dev, D, Hq, Hk):
    from dspark_rocm import ops

    M, pos0, cap = 16, 16384, 16384 + 64
    g = torch.Generator(device=dev)
    g.manual_seed(D)
    q = torch.randn((M, Hq * D), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((M, Hk * D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((M, Hk * D), generator=g, device=dev).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
    kc = torch.zeros((Hk, cap, D), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    qo = torch.empty((Hq, M, D), dtype=torch.bfloat16, device=dev)
    ops.qk_norm_rope_kv(q, k, v, qw, kw, heads=Hq, kv_heads=Hk, head_dim=D, eps=1e-6, rope_base=1e6, pos0=pos0,
                        q_out=qo, k_cache=kc, v_cache=vc)
    pos = np.arange(pos0, pos0 + M)
    qr = model_ref.rope(model_ref.rmsnorm(_np(q).reshape(M, Hq, D).transpose(1, 0, 2), _np(qw), 1e-6), pos, 1e6)
    kr = model_ref.rope(model_ref.rmsnorm(_np(k).reshape(M, Hk, D).transpose(1, 0, 2), _np(kw), 1e-6), pos, 1e6)
    tol = 2 ** -6 * max(np.abs(qr).max(), 1.0)                      # bf16 ulps of the fp32 angle path
    assert np.abs(_np(qo) - qr).max() <= tol
    assert np.abs(_np(kc[:, pos0:pos0 + M]) - kr).max() <= tol
    assert np.array_equal(_np(vc[:, pos0:pos0 + M]), _np(v).reshape(M, Hk, D).transpose(1, 0, 2))
    assert not kc[:, :pos0].any() and not kc[:, pos0 + M:].any()   # nothing outside the block


@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("base", [1e4, 1e6])
def test_rope_kernel_frequency_schedule(dev, D, base):
    """The closed-form RoPE KAT (tests/_util.rope_kat_errors) through the kernel. With unit q/k
    norm weights and eps 0, RMSNorm maps e_i to r0 * e_i, r0 = bf16(sqrt(D)); dividing r0 out
    leaves the rotation of e_i at position p, for the q output and the cached k alike."""
    from dspark_rocm import ops

    ones = torch.ones(D, dtype=torch.bfloat16, device=dev)
    r0 = float(model_ref.bf(np.full(1, np.sqrt(D), np.float32))[0])

    def rope_fn(x, pos, b):
        p = int(pos[0])
        xv = torch.from_numpy(np.ascontiguousarray(x.reshape(1, D))).to(dev).to(torch.bfloat16)
        kc = torch.zeros((1, p + 1, D), dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        qo = torch.empty((1, 1, D), dtype=torch.bfloat16, device=dev)
        ops.qk_norm_rope_kv(xv, xv, xv, ones, ones, heads=1, kv_heads=1, head_dim=D, eps=0.0, rope_base=b, pos0=p,
                            q_out=qo, k_cache=kc, v_cache=vc)
        q, k = _np(qo).reshape(D), _np(kc[0, p])
        assert np.array_equal(q, k)
        return q / r0

    assert rope_kat_errors(rope_fn, D, base) <= ROPE_KAT_TOL


def _argmax_ref(rows: np.ndarray) -> list[int]:
    """First index of the maximum; NaN never chosen (an all-NaN row gives 0)."""
    out = []
    for r in rows:
        r = np.where(np.isnan(r), -np.inf, r)
        out.append(int(np.argmax(r)))
    return out


@pytest.mark.parametrize("M,V", [(16, 151936), (6, 8192), (3, 8193), (2, 5), (16, 100003), (1, 32000)])
def test_argmax_accept_fused(dev, M, V):
    """One launch of argmax + greedy accept equals argmax_rows followed by greedy_accept: ties
    across the workgroups' chunks go to the first index, NaN is never chosen, the last element
    and a ragged tail count; repeated calls and graph replays leave the counter at zero."""
    from dspark_rocm import ops

    g = torch.Generator(device=dev)
    g.manual_seed(M * 7 + V)
    ld = (V + 7) // 8 * 8                                           # rows 16-byte aligned, V ragged
    logits = torch.randn((M, ld), generator=g, device=dev).to(torch.bfloat16)[:, :V]
    if V > 9000:
        logits[0, 8200] = 40.0
        logits[0, V - 3] = 40.0                                     # tie across chunks: 8200 wins
        logits[M - 1, V - 1] = 45.0                                 # the last element
    if M > 2:
        logits[1] = float("nan")                                    # all NaN -> token 0
        logits[2, : V // 2] = float("nan")                          # NaN never chosen
        logits[2, V // 2] = 30.0
    want = _argmax_ref(_np(logits).astype(np.float64))
    assert ops.argmax_rows(logits).cpu().tolist() == want
    ws = torch.zeros(ops.argmax_accept_workspace_bytes(M, V), dtype=torch.uint8, device=dev)
    tt = torch.empty(M, dtype=torch.int32, device=dev)
    n = torch.empty(1, dtype=torch.int32, device=dev)
    for k in range(min(M - 1, 3) + 1):                              # drafts matching k leading tokens
        draft = want[:k] + ([want[k] + 1] if k < M - 1 else [])
        d = torch.tensor(draft, dtype=torch.int32, device=dev)
        tt.fill_(-1)
        ops.argmax_accept(logits, d, tt, n, ws)
        assert tt.cpu().tolist() == want
        assert int(n.item()) == verify_ref.greedy_accept(draft, want)[0]
        assert int(ops.greedy_accept(d, tt).item()) == int(n.item())
        assert not ws[:256].any()
    d = torch.tensor(want[: M - 1], dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.argmax_accept(logits, d, tt, n, ws)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        ops.argmax_accept(logits, d, tt, n, ws)
    for _ in range(3):
        tt.fill_(-1)
        n.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert tt.cpu().tolist() == want and int(n.item()) == M - 1
        assert not ws[:256].any()


def test_swiglu_argmax_accept_kernels(dev):
    from dspark_rocm import ops

    g = torch.Generator(device=dev)
    g.manual_seed(1)
    a = (3 * torch.randn((16, 4096), generator=g, device=dev)).to(torch.bfloat16)
    b = torch.randn((16, 4096), generator=g, device=dev).to(torch.bfloat16)
    assert np.array_equal(_np(ops.swiglu(a, b)), moe_ref.swiglu(_np(a), _np(b)))
    logits = torch.randn((6, 151936), generator=g, device=dev).to(torch.bfloat16)
    logits[2, 77] = 50.0
    logits[2, 9000] = 50.0                                          # tie: the first index wins
    logits[4, 151935] = 60.0                                        # the last element
    tt = ops.argmax_rows(logits)
    want = [int(np.argmax(r)) for r in _np(logits)]
    assert tt.cpu().tolist() == want and want[2] == 77 and want[4] == 151935
    for draft, tts in (([5, 6, 7], [5, 6, 9, 1]), ([1, 2], [1, 2, 3]), ([4], [5, 6]), ([], [8])):
        n = ops.greedy_accept(torch.tensor(draft, dtype=torch.int32), torch.tensor(tts, dtype=torch.int32, device=dev))
        assert int(n.item()) == verify_ref.greedy_accept(draft, tts)[0]


def test_fused_verify_matches_oracle_with_rollback(dev):
    from dspark_rocm.model import Target

    model = tiny_model(dev, seed=5)
    ref = to_ref(model)
    tgt = Target(model)
    cache = tgt.make_cache(128)
    r = np.random.Generator(np.random.PCG64(0))
    blocks = [r.integers(0, 512, n).tolist() for n in (16, 9, 16, 1, 12)]
    rejects = [0, 5, 15, 0, 3]
    for ids, rej in zip(blocks, rejects):
        got, _ = tgt.verify(torch.tensor([ids]), cache)
        want = ref.forward(ids)
        # whole forward: each op is within its kernel's bar; ~10 bf16 rounding points per layer
        # compound, so the logits get 5e-2 * RMS and the greedy tokens must agree wherever the
        # top-2 margin exceeds that error
        err, _ = assert_rms_close(_np(got[0]), want, 5e-2, f"verify block of {len(ids)}")
        top2 = np.sort(want, axis=-1)[:, -2:]
        clear = (top2[:, 1] - top2[:, 0]) > 2 * err
        assert np.array_equal(_np(got[0]).argmax(-1)[clear], want.argmax(-1)[clear])
        tgt.rollback(cache, rej)
        ref.trim(rej)
        assert cache[0].offset == ref.offset


def test_rollback_then_verify_is_bitwise_a_fresh_prefix(dev):
    from dspark_rocm.model import Target

    model = tiny_model(dev, seed=6)
    tgt = Target(model)
    a = tgt.make_cache(64)
    tgt.verify(torch.tensor([list(range(10, 26))]), a)              # 16 rows
    tgt.rollback(a, 11)                                              # keep 5
    la, _ = tgt.verify(torch.tensor([[1, 2, 3, 4]]), a)
    b = tgt.make_cache(64)
    tgt.verify(torch.tensor([list(range(10, 15))]), b)
    lb, _ = tgt.verify(torch.tensor([[1, 2, 3, 4]]), b)
    assert torch.equal(la, lb)


def test_module_path_under_scopes_matches_fused(dev):
    from dspark_rocm import multirow_attn as mra
    from dspark_rocm import small_m_qmm as sm
    from dspark_rocm.model import Target

    model = tiny_model(dev, seed=7)
    tgt = Target(model)
    ids = torch.tensor([[3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5, 8, 9, 7, 9, 3]])      # 16 rows: attention eligible
    ca, cb = tgt.make_cache(64), tgt.make_cache(64)
    fused, _ = tgt.verify(ids, ca)
    a = model.args
    cfg = mra.MultirowConfig((mra.Window(a.num_attention_heads, a.num_key_value_heads, a.head_dim, min_q=2,
                                         max_q=16, min_kv=16),))
    ids_all = sm.ids_for_shapes([sm.shape_key(m) for m in model.modules() if sm.eligible(m)], model)
    with sm.small_m_matmul(ids_all), mra.multirow_attention(cfg), torch.no_grad():
        mod = model(ids.to(dev), cb)
    assert_rms_close(_np(mod[0]), _np(fused[0]), 5e-2, "module path vs fused")


def test_speculative_trace_is_lossless_with_expected_accept_length(dev):
    """Drafts are the plain-greedy continuation with seeded corruptions; every round must
    commit exactly the greedy tokens and accept up to the first corrupted draft token."""
    from dspark_rocm.model import Target, greedy_generate

    model = tiny_model(dev, seed=8)
    tgt = Target(model)
    prompt = [11, 22, 33, 44, 55]
    steps = 60
    greedy = greedy_generate(tgt, prompt, steps + 16)
    r = np.random.Generator(np.random.PCG64(12))
    cache = tgt.make_cache(len(prompt) + steps + 40)
    for i in range(0, len(prompt), 16):
        tgt.verify(torch.tensor([prompt[i:i + 16]]), cache)
    out = [greedy[0]]
    rounds, expected_acc = 0, []
    while len(out) < steps:
        cap = int(r.integers(1, 8))
        truth = greedy[len(out):len(out) + cap]
        draft = [t if r.random() > 0.3 else (t + 1) % 512 for t in truth]
        n_expect = next((j for j, (d, t) in enumerate(zip(draft, truth)) if d != t), len(draft))
        n, committed, _ = tgt.greedy_round(out[-1], draft, cache)
        assert n == n_expect, (rounds, draft, truth)
        out += committed
        expected_acc.append(n + 1)
        rounds += 1
        assert cache[0].offset == len(prompt) + len(out) - 1
    assert out[:steps] == greedy[:steps]
    # the first token came from the prompt's forward; the rounds committed the rest
    assert verify_ref.mean_accept_len(sum(expected_acc), rounds) == (len(out) - 1) / rounds


def test_verify_tap_returns_the_tapped_hidden_states(dev):
    """Target.verify(ids, cache, tap) -> (logits, fused [1, M, n_tap * H]): the residual stream
    after each tapped layer in layer order, whatever the order, duplicates or out-of-range
    entries of ``tap`` (target.py:208-220, :642-677). The tap changes no logit bit; each column
    block is bitwise the block a one-layer tap returns; against the oracle's tapped forward and
    the module path's capture within the multi-layer forward's bar per block (5e-2 x RMS, as
    for the logits: the stream is bf16 after every layer, and one ulp of its largest values is
    ~3% of its RMS); ``tap=None`` returns None; the prefill chunk returns the same capture
    through the module path (target.py:435-465)."""
    from dspark_rocm.model import Target, tap_layers

    model = tiny_model(dev, seed=13, num_hidden_layers=4)
    H = model.args.hidden_size
    tgt = Target(model)
    tap = [3, 1, 1, 9, -2]
    assert tap_layers(tap, 4) == (1, 3)
    r = np.random.Generator(np.random.PCG64(14))
    prefix = r.integers(0, 512, 20).tolist()
    block = r.integers(0, 512, 12).tolist()
    runs = {}
    for key, t in (("none", None), ("both", tap), ("l1", [1]), ("l3", [3])):
        cache = tgt.make_cache(64)
        tgt.verify(torch.tensor([prefix[:16]]), cache)
        tgt.verify(torch.tensor([prefix[16:]]), cache)
        logits, fused = tgt.verify(torch.tensor([block]), cache, t)
        runs[key] = (logits.clone(), None if fused is None else fused.clone())
    assert runs["none"][1] is None
    fused = runs["both"][1]
    assert fused.shape == (1, 12, 2 * H) and fused.dtype == torch.bfloat16
    for key in ("both", "l1", "l3"):
        assert torch.equal(runs[key][0], runs["none"][0]), key
    assert torch.equal(fused[..., :H], runs["l1"][1]) and torch.equal(fused[..., H:], runs["l3"][1])

    ref = to_ref(model)
    ref.forward(prefix)
    ref.forward(block, tap=tap)
    want = ref.fused
    assert want.shape == (12, 2 * H)
    for j in range(2):
        assert_rms_close(_np(fused[0, :, j * H:(j + 1) * H]), want[:, j * H:(j + 1) * H], 5e-2, f"tap block {j}")
    # the module path (Target.run) and a prefill chunk capture the same stream
    cm = tgt.make_cache(64)
    tgt.prefill(torch.tensor([prefix]), cm)
    with torch.no_grad():
        logits_m, fused_m = tgt.run(torch.tensor([block]), cm, tap)
    assert fused_m.shape == fused.shape
    assert_rms_close(_np(fused_m[0]), _np(fused[0]), 5e-2, "module path capture")
    cp = tgt.make_cache(64)
    with torch.no_grad():
        none, fused_p = tgt.prefill(torch.tensor([prefix + block]), cp, tap)
        lp, nofused = tgt.prefill(torch.tensor([block[:3]]), cp, want_logits=True)
    assert none is None and nofused is None and lp.shape == (1, 1, model.args.vocab_size)
    assert fused_p.shape == (1, 32, 2 * H)
    assert_rms_close(_np(fused_p[0, 20:]), want, 5e-2, "prefill capture")


def test_speculative_trace_feeds_the_drafter_its_context_rows(dev):
    """The DSpark loop's context update (generate.py:1547, :1590-1593): every round hands
    fused[:, :n + 1] (the tapped states of [pending, accepted drafts]) to the drafter. A stub
    update_context checks each call's shape and offset; over the whole trace the rows it
    received are the oracle's tapped stream over the committed tokens, position for position
    (within the multi-layer forward's 5e-2 x RMS bar)."""
    from dspark_rocm.model import Target

    model = tiny_model(dev, seed=15, num_hidden_layers=3)
    H = model.args.hidden_size
    tgt = Target(model)
    tap = [0, 2]
    r = np.random.Generator(np.random.PCG64(16))
    prompt = r.integers(0, 512, 9).tolist()
    cache = tgt.make_cache(128)
    logits, _ = tgt.verify(torch.tensor([prompt]), cache, tap)
    out = [int(torch.argmax(logits[0, -1].float()))]
    received = []

    def update_context(rows, ctx_offset):
        assert rows.shape[0] == 1 and rows.shape[2] == len(tap) * H
        assert ctx_offset == len(prompt) + sum(x.shape[1] for x in received)
        received.append(rows.clone())

    n_cached = len(prompt)
    while len(out) < 40:
        draft = [int(t) for t in r.integers(0, 512, int(r.integers(0, 6)))]
        n, committed, ctx = tgt.greedy_round(out[-1], draft, cache, tap)
        assert ctx.shape == (1, n + 1, len(tap) * H)
        update_context(ctx, n_cached)
        n_cached += n + 1
        out += committed
    got = torch.cat(received, dim=1)[0]
    ref = to_ref(model)
    ref.forward(prompt + out[:-1], tap=tap)
    want = ref.fused[len(prompt):]
    assert got.shape == want.shape
    assert_rms_close(_np(got), want, 5e-2, "context rows over the trace")


def test_packed_engine_is_bitwise_the_reference_layout_engine(dev):
    """The fused step reading every projection from the packed qmm form (hidden 512 and
    intermediate 1024, so all seven projections and the lm_head are packable; gate and up as the
    fused gate / up / SwiGLU pair) produces the same logits, bit for bit, as the step reading the
    reference layout (gate, up and the SwiGLU kernel), over blocks with rollback."""
    from dspark_rocm.model import Target

    model = tiny_model(dev, seed=9, hidden_size=512, intermediate_size=1024)
    packed, plain = Target(model, packed=True), Target(model, packed=False)
    layers = model.args.num_hidden_layers
    assert len(packed.engine._packed) == 5 * layers + 1 and len(packed.engine._swiglu) == layers
    assert not plain.engine._packed and not plain.engine._swiglu
    ca, cb = packed.make_cache(96), plain.make_cache(96)
    r = np.random.Generator(np.random.PCG64(4))
    for n, rej in ((16, 3), (7, 0), (16, 15)):
        ids = torch.tensor([r.integers(0, 512, n).tolist()])
        la, _ = packed.verify(ids, ca)
        lb, _ = plain.verify(ids, cb)
        assert torch.equal(la, lb)
        packed.rollback(ca, rej)
        plain.rollback(cb, rej)


def test_captured_step_replays_after_deeper_eager_steps(dev):
    """A verify step captured at a short cache length stays correct when eager steps at a much
    deeper length (whose attention plan needs more split-KV partials) run on the same stream
    between replays: the engine's workspaces are sized at construction for any length, so no
    buffer a graph holds is replaced. Every replay is bitwise the eager result at the short
    length."""
    from dspark_rocm.model import Target

    model = tiny_model(dev, seed=10)
    tgt = Target(model)
    e = tgt.engine
    cache = tgt.make_cache(4096 + 64)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    for c in cache:
        c.keys.normal_(generator=g)
        c.values.normal_(generator=g)
    M, short, deep = 16, 600, 4000
    a = model.args
    from dspark_rocm import ops
    assert ops.verify_attention_blocks(1, a.num_attention_heads, a.num_key_value_heads, M, a.head_dim, deep + M) > \
        ops.verify_attention_blocks(1, a.num_attention_heads, a.num_key_value_heads, M, a.head_dim, short + M) > 1
    e.ids[:M].copy_(torch.randint(0, a.vocab_size, (M,), generator=g, device=dev))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        e.step(M, cache, short)
        want = e.logits[:M].clone()
        e.step(M, cache, short)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        e.step(M, cache, short)
    torch.cuda.synchronize()
    for rep in range(3):
        with torch.cuda.stream(s):
            e.step(M, cache, deep + 8 * rep)
            deep_logits = e.logits[:M].clone()
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(e.logits[:M], want), rep
        assert not torch.equal(deep_logits, want)
