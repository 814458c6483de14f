"""Dense qwen3-style target and its verify forward on the gfx950 kernels.

The reference verifies a draft by running its target's forward over ``[anchor] + draft``
rows against the KV cache (``Target.verify``, target.py:642-677 -> ``run`` / ``_body_mlxlm`` /
``_head_mlxlm``, :187-221, :347-354): mlx-lm's DecoderLayer stack (third-party) with every
projection a ``QuantizedLinear`` and every attention call ``mx.fast.scaled_dot_product_attention``.

Two forwards of the same weights live here:

* :meth:`DenseModel.forward` — the module path, op for op the mlx-lm layer on torch tensors:
  its projections are :class:`~dspark_rocm.nn.QuantizedLinear` calls and its attention goes
  through :func:`dspark_rocm.fast.scaled_dot_product_attention`, so the reference's scopes
  (``small_m_matmul``, ``multirow_attention``, ``sdpa_split``) route it exactly as they route
  mlx-lm. Norms and RoPE are torch ops with the same bf16 rounding points as the kernels.
* :class:`VerifyEngine` — the MI355X verify step: per layer one fused residual-add + RMSNorm,
  one q/k/v qmm launch, one q/k-norm + RoPE + cache-write kernel, split-KV attention writing
  o_proj's input rows directly, the o qmm, residual-add + RMSNorm, one fused gate/up/SwiGLU
  qmm launch (packed weights; else a gate/up launch and the SwiGLU kernel), the down qmm; then
  the final norm, lm_head, and the device argmax with greedy accept (one launch). All buffers, the qmm and attention
  workspaces included, are preallocated for up to ``max_rows`` rows and any cache length, so a
  step can be captured in a hipGraph and replayed after steps at other depths.

:class:`Target` mirrors the reference's ``verify`` / ``rollback`` / ``make_cache`` surface and
the greedy round (generate.py:1544-1593).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import nn

from . import fast, ops
from ._lib import load as _lib_load
from .kv_cache import KVCache, QuantizedKVCache
from .nn import QuantizedLinear


@dataclass(frozen=True)
class ModelArgs:
    hidden_size: int
    num_hidden_layers: int
    intermediate_size: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    vocab_size: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    bits: int = 8
    lm_head_bits: int = 8


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """``bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)`` (fp32 statistics)."""
    xf = x.float()
    inv = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return ((xf * inv).to(torch.bfloat16).float() * w.float()).to(torch.bfloat16)


def rope(x: torch.Tensor, pos0: int, base: float) -> torch.Tensor:
    """Non-traditional RoPE over the last dim of x [..., L, D] at positions pos0..pos0+L-1."""
    D = x.shape[-1]
    half = D // 2
    i = torch.arange(half, device=x.device, dtype=torch.float32)
    inv_freq = torch.exp2(-(2.0 * i / D) * math.log2(base))
    pos = torch.arange(pos0, pos0 + x.shape[-2], device=x.device, dtype=torch.float32)
    ang = pos[:, None] * inv_freq[None, :]
    c, s = torch.cos(ang), torch.sin(ang)
    x1, x2 = x[..., :half].float(), x[..., half:].float()
    return torch.cat([(x1 * c - x2 * s).to(torch.bfloat16), (x1 * s + x2 * c).to(torch.bfloat16)], dim=-1)


class Attention(nn.Module):
    def __init__(self, args: ModelArgs, q, k, v, o, q_norm, k_norm):
        super().__init__()
        self.args = args
        self.q_proj, self.k_proj, self.v_proj, self.o_proj = q, k, v, o
        self.register_buffer("q_norm", q_norm)
        self.register_buffer("k_norm", k_norm)

    def forward(self, x: torch.Tensor, cache: KVCache) -> torch.Tensor:
        a = self.args
        B, L, _ = x.shape
        hq, hk, d = a.num_attention_heads, a.num_key_value_heads, a.head_dim
        q = rms_norm(self.q_proj(x).reshape(B, L, hq, d), self.q_norm, a.rms_norm_eps).transpose(1, 2)
        k = rms_norm(self.k_proj(x).reshape(B, L, hk, d), self.k_norm, a.rms_norm_eps).transpose(1, 2)
        v = self.v_proj(x).reshape(B, L, hk, d).transpose(1, 2)
        q = rope(q, cache.offset, a.rope_theta)
        k = rope(k, cache.offset, a.rope_theta)
        keys, values = cache.update_and_fetch(k, v)
        mask = "causal" if L > 1 else None
        if hasattr(cache, "bits"):
            # mlx-lm's attention helper dispatches per cache: a quantized cache takes
            # quantized_scaled_dot_product_attention over its (words, scales, biases) triples
            out = fast.quantized_scaled_dot_product_attention(q.contiguous(), keys, values, scale=d ** -0.5,
                                                              mask=mask, group_size=cache.group_size,
                                                              bits=cache.bits)
        else:
            out = fast.scaled_dot_product_attention(q.contiguous(), keys, values, scale=d ** -0.5, mask=mask)
        return self.o_proj(out.transpose(1, 2).reshape(B, L, hq * d))


class MLP(nn.Module):
    def __init__(self, gate, up, down):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = gate, up, down

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        g = self.gate_proj(x)
        return self.down_proj((g * torch.sigmoid(g)) * self.up_proj(x))


class DecoderLayer(nn.Module):
    def __init__(self, args: ModelArgs, attn: Attention, mlp: MLP, input_norm, post_norm):
        super().__init__()
        self.args = args
        self.self_attn, self.mlp = attn, mlp
        self.register_buffer("input_layernorm", input_norm)
        self.register_buffer("post_attention_layernorm", post_norm)

    def forward(self, x: torch.Tensor, cache: KVCache) -> torch.Tensor:
        eps = self.args.rms_norm_eps
        h = x + self.self_attn(rms_norm(x, self.input_layernorm, eps), cache)
        return h + self.mlp(rms_norm(h, self.post_attention_layernorm, eps))


class DenseModel(nn.Module):
    def __init__(self, args: ModelArgs, embed: torch.Tensor, layers: list[DecoderLayer], norm: torch.Tensor,
                 lm_head: QuantizedLinear):
        super().__init__()
        self.args = args
        self.register_buffer("embed_tokens", embed)
        self.layers = nn.ModuleList(layers)
        self.register_buffer("norm", norm)
        self.lm_head = lm_head

    @classmethod
    def random(cls, args: ModelArgs, *, device, seed: int = 0) -> "DenseModel":
        """Random-init weights of this architecture (packed affine weights drawn directly in the
        packed domain; norm weights near 1; bf16 embedding table)."""
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        H, I, hq, hk, d = (args.hidden_size, args.intermediate_size, args.num_attention_heads,
                           args.num_key_value_heads, args.head_dim)

        def lin(n, k, bits=args.bits):
            return QuantizedLinear.random(n, k, bits=bits, device=device, generator=g)

        def normw(n):
            return (1.0 + 0.1 * torch.randn(n, generator=g, device=device)).to(torch.bfloat16)

        layers = []
        for _ in range(args.num_hidden_layers):
            attn = Attention(args, lin(hq * d, H), lin(hk * d, H), lin(hk * d, H), lin(H, hq * d), normw(d), normw(d))
            layers.append(DecoderLayer(args, attn, MLP(lin(I, H), lin(I, H), lin(H, I)), normw(H), normw(H)))
        embed = torch.randn((args.vocab_size, H), generator=g, device=device).to(torch.bfloat16)
        return cls(args, embed, layers, normw(H), lin(args.vocab_size, H, args.lm_head_bits))

    def make_cache(self, capacity: int = 0, kv_bits: int | None = None, kv_group_size: int = 64) -> list:
        """One KV cache per layer; with ``kv_bits`` (4 or 8) every layer's cache is quantized
        (target.py:166-184: a dense target replaces each plain cache by mlx-lm's
        QuantizedKVCache)."""
        a = self.args
        dev = self.embed_tokens.device
        if kv_bits:
            return [QuantizedKVCache(1, a.num_key_value_heads, a.head_dim, bits=kv_bits, group_size=kv_group_size,
                                     device=dev, capacity=capacity) for _ in range(a.num_hidden_layers)]
        return [KVCache(1, a.num_key_value_heads, a.head_dim, device=dev, capacity=capacity)
                for _ in range(a.num_hidden_layers)]

    def body(self, ids: torch.Tensor, cache: list[KVCache], tap=None):
        """ids [1, L] -> (final-normed hidden states [1, L, H], fused | None), the module path.
        ``fused`` [1, L, n_tap * H] concatenates the residual stream after every decoder layer
        whose index is in ``tap``, in layer order (target.py:208-220 ``_body_mlxlm``); ``tap``
        None skips the capture."""
        slots = tap_layers(tap, len(self.layers))
        h = self.embed_tokens[ids]
        captured = []
        for i, (layer, c) in enumerate(zip(self.layers, cache)):
            h = layer(h, c)
            if i in slots:
                captured.append(h)
        fused = None
        if tap is not None:
            fused = torch.cat(captured, dim=-1) if captured else h.new_empty((*h.shape[:-1], 0))
        return rms_norm(h, self.norm, self.args.rms_norm_eps), fused

    def forward(self, ids: torch.Tensor, cache: list[KVCache]) -> torch.Tensor:
        """ids [1, L] -> logits [1, L, V] (the module path)."""
        return self.lm_head(self.body(ids, cache)[0])


def tap_layers(tap, n_layers: int) -> tuple[int, ...]:
    """The layers a hidden-state tap captures, in layer order: the reference tests each layer
    index against the tap set while it walks the stack (target.py:210-219), so the order of
    ``tap``, duplicates and indices outside the stack do not matter."""
    if tap is None:
        return ()
    return tuple(sorted({int(i) for i in tap if 0 <= int(i) < n_layers}))


PREFILL_CHUNK = 2048    # a long prompt prefills in pieces of this many rows (generate.py:1026)


class VerifyEngine:
    """Preallocated fused verify step for up to ``max_rows`` rows (batch 1). With ``packed``,
    every projection whose K is a multiple of 512 is held (also) in the MI355X packed qmm form
    (``ops.qmm_pack``, packed once here) and multiplied from it; products are bit-identical to
    the reference layout's. Each MLP's gate and up projections are packed as one pair
    (``ops.qmm_pack_swiglu``) and run as one fused gate / up / SwiGLU launch, bit-identical to
    the two products followed by SwiGLU when the intermediate size is a multiple of 64."""

    def __init__(self, model: DenseModel, max_rows: int = 16, packed: bool = True):
        a = model.args
        self.model, self.args, self.max_rows = model, a, max_rows
        self._packed: dict[int, ops.PackedQmm] = {}
        self._swiglu: dict[int, ops.PackedSwiGLU] = {}
        if packed:
            mods = [model.lm_head]
            for layer in model.layers:
                at, mlp = layer.self_attn, layer.mlp
                mods += [at.q_proj, at.k_proj, at.v_proj, at.o_proj, mlp.down_proj]
                g, u = mlp.gate_proj, mlp.up_proj
                n, k = g.weight.shape[0], g.weight.shape[1] * 32 // g.bits
                if g.bits == u.bits and g.weight.shape == u.weight.shape and ops.qmm_packable(n, k, g.bits):
                    self._swiglu[id(mlp)] = ops.qmm_pack_swiglu((g.weight, g.scales, g.biases),
                                                                (u.weight, u.scales, u.biases), bits=g.bits)
                else:
                    mods += [g, u]
            for mod in mods:
                n, k = mod.weight.shape[0], mod.weight.shape[1] * 32 // mod.bits
                if ops.qmm_packable(n, k, mod.bits):
                    self._packed[id(mod)] = ops.qmm_pack(mod.weight, mod.scales, mod.biases, bits=mod.bits)
        dev = model.embed_tokens.device
        H, I, hq, hk, d = (a.hidden_size, a.intermediate_size, a.num_attention_heads, a.num_key_value_heads,
                           a.head_dim)
        bf = torch.bfloat16
        e = lambda *s: torch.empty(s, dtype=bf, device=dev)
        self.h, self.r, self.y = e(max_rows, H), e(max_rows, H), e(max_rows, H)
        self.q, self.k, self.v = e(max_rows, hq * d), e(max_rows, hk * d), e(max_rows, hk * d)
        self.qatt = e(1, hq, max_rows, d)
        self.att = e(max_rows, hq * d)
        self.g, self.u, self.hm = e(max_rows, I), e(max_rows, I), e(max_rows, I)
        self.logits = e(max_rows, a.vocab_size)
        self.ids = torch.zeros(max_rows, dtype=torch.int64, device=dev)
        self.tt = torch.zeros(max_rows, dtype=torch.int32, device=dev)
        self.draft = torch.zeros(max(max_rows - 1, 1), dtype=torch.int32, device=dev)
        self.n_acc = torch.zeros(1, dtype=torch.int32, device=dev)
        # The engine's own workspaces, sized once for every launch of a step at up to max_rows
        # rows and any cache length, so a captured step never sees them move.
        self.qmm_ws = ops.new_qmm_workspace(dev, self._qmm_workspace_need())
        self.accept_ws = torch.zeros(max(ops.argmax_accept_workspace_bytes(max_rows, a.vocab_size), 256),
                                     dtype=torch.uint8, device=dev)
        # hidden-state tap: the residual stream after each tapped layer, written in place by the
        # residual add that forms it (no copy), [max_rows, n_tap * H]; see set_tap
        self.tap: tuple[int, ...] = ()
        self.fused = e(max_rows, 0)
        self.attn_ws = torch.empty(max(ops.attention_workspace_bound(1, hq, hk, d, max_rows), 16), dtype=torch.uint8,
                                   device=dev)

    def _qmm_workspace_need(self) -> int:
        a, m, M = self.args, self.model, self.max_rows
        need = []
        for layer in m.layers:
            at, mlp = layer.self_attn, layer.mlp
            groups = [[at.q_proj, at.k_proj, at.v_proj], [at.o_proj], [mlp.down_proj]]
            pair = self._swiglu.get(id(mlp))
            if pair is not None:
                need.append(int(_lib_load().dspark_qmm_swiglu_packed_workspace(pair.n, pair.k, M, pair.bits, 64)))
            else:
                groups.append([mlp.gate_proj, mlp.up_proj])
            for mods in groups:
                k = mods[0].weight.shape[1] * 32 // mods[0].bits
                need.append(ops.qmm_launch_workspace_bytes(M, k, [mod.weight.shape[0] for mod in mods], mods[0].bits))
        lm = m.lm_head
        need.append(ops.qmm_launch_workspace_bytes(M, a.hidden_size, [lm.weight.shape[0]], lm.bits))
        return max(need)

    def set_tap(self, tap) -> tuple[int, ...]:
        """Select the layers whose residual-stream output the step writes into ``self.fused``
        (column block j holds layer ``self.tap[j]``). Reallocates the buffer when the number of
        tapped layers changes, so call it before capturing a step in a graph."""
        slots = tap_layers(tap, self.args.num_hidden_layers)
        if len(slots) != self.fused.shape[1] // self.args.hidden_size:
            self.fused = torch.empty((self.max_rows, len(slots) * self.args.hidden_size), dtype=torch.bfloat16,
                                     device=self.h.device)
        self.tap = slots
        return slots

    def _qmm(self, x: torch.Tensor, mods, outs) -> None:
        """One launch of ``x @ W^T`` for the modules ``mods`` (same K and bits) into ``outs``."""
        packs = [self._packed.get(id(mod)) for mod in mods]
        if all(p is not None for p in packs):
            ops.quantized_matmul_packed_multi([x], packs, outs=outs, workspace=self.qmm_ws)
        else:
            ops.quantized_matmul_multi([x], [mod.weight for mod in mods], [mod.scales for mod in mods],
                                       [mod.biases for mod in mods], bits=mods[0].bits, outs=outs,
                                       workspace=self.qmm_ws)

    def step(self, M: int, cache: list[KVCache], pos0: int, *, accept: bool = False) -> torch.Tensor:
        """Run the forward over ``self.ids[:M]`` at cache positions pos0..pos0+M-1 (caches
        already reserved); logits in ``self.logits[:M]``; with ``accept``, also the target
        tokens ``self.tt[:M]`` and the accepted count ``self.n_acc`` for ``self.draft[:M-1]``;
        the tapped layers' residual streams (``set_tap``) in ``self.fused[:M]``.
        Enqueues kernels only (graph-capturable for a fixed pos0)."""
        a, m = self.args, self.model
        hq, hk, d, eps = a.num_attention_heads, a.num_key_value_heads, a.head_dim, a.rms_norm_eps
        h, r, y = self.h[:M], self.r[:M], self.y[:M]
        torch.index_select(m.embed_tokens, 0, self.ids[:M], out=h)
        L = pos0 + M
        H = a.hidden_size
        slot = {li: j for j, li in enumerate(self.tap)}

        def stream_out(li: int) -> torch.Tensor:
            """Where the residual add that completes layer ``li`` writes the stream: its tap
            column block when tapped (the next add reads it from there), else ``h``."""
            j = slot.get(li)
            return h if j is None else self.fused[:M, j * H:(j + 1) * H]

        hcur = h
        qatt = self.qatt[:, :, :M]
        if M != self.max_rows:
            qatt = self.qatt.view(-1)[:hq * M * d].view(1, hq, M, d)
        for li, (layer, c) in enumerate(zip(m.layers, cache)):
            at, mlp = layer.self_attn, layer.mlp
            if li == 0:
                ops.rmsnorm(hcur, layer.input_layernorm, eps, out=y)
            else:
                dst = stream_out(li - 1)
                ops.rmsnorm(hcur, layer.input_layernorm, eps, residual=r, h_out=dst, out=y)
                hcur = dst
            self._qmm(y, [at.q_proj, at.k_proj, at.v_proj], [self.q[:M], self.k[:M], self.v[:M]])
            att = self.att[:M]
            ostr = (M * hq * d, d, hq * d)
            if hasattr(c, "bits"):      # quantized cache: rows quantized as written, attention on the triples
                ops.qk_norm_rope_kv_quantized(self.q[:M], self.k[:M], self.v[:M], at.q_norm, at.k_norm, heads=hq,
                                              kv_heads=hk, head_dim=d, eps=eps, rope_base=a.rope_theta, pos0=pos0,
                                              q_out=qatt[0], k_cache=tuple(t[0] for t in c.keys),
                                              v_cache=tuple(t[0] for t in c.values), bits=c.bits,
                                              group_size=c.group_size)
                ops.verify_attention_quantized(qatt, tuple(t[:, :, :L] for t in c.keys),
                                               tuple(t[:, :, :L] for t in c.values), scale=d ** -0.5, causal=M > 1,
                                               bits=c.bits, group_size=c.group_size, out=att, out_strides=ostr,
                                               workspace=self.attn_ws)
            else:
                ops.qk_norm_rope_kv(self.q[:M], self.k[:M], self.v[:M], at.q_norm, at.k_norm, heads=hq,
                                    kv_heads=hk, head_dim=d, eps=eps, rope_base=a.rope_theta, pos0=pos0,
                                    q_out=qatt[0], k_cache=c.keys[0], v_cache=c.values[0])
                ops.verify_attention_into(qatt, c.keys[:, :, :L], c.values[:, :, :L], att, ostr, scale=d ** -0.5,
                                          causal=M > 1, workspace=self.attn_ws)
            self._qmm(att, [at.o_proj], [r])
            ops.rmsnorm(hcur, layer.post_attention_layernorm, eps, residual=r, h_out=h, out=y)
            hcur = h
            pair = self._swiglu.get(id(mlp))
            if pair is not None:
                ops.quantized_swiglu_packed(y, pair, out=self.hm[:M], workspace=self.qmm_ws)
            else:
                self._qmm(y, [mlp.gate_proj, mlp.up_proj], [self.g[:M], self.u[:M]])
                ops.swiglu(self.g[:M], self.u[:M], out=self.hm[:M])
            self._qmm(self.hm[:M], [mlp.down_proj], [r])
        ops.rmsnorm(hcur, m.norm, eps, residual=r, h_out=stream_out(len(m.layers) - 1), out=y)
        lm = m.lm_head
        logits = self.logits[:M]
        self._qmm(y, [lm], [logits])
        if accept:
            ops.argmax_accept(logits, self.draft[:M - 1], self.tt[:M], self.n_acc, self.accept_ws)
        return logits


class Target:
    """The reference's Target surface for a dense model: ``make_cache``, ``verify``,
    ``plain``, ``rollback`` (target.py:166-184, :642-696), plus the greedy round."""

    def __init__(self, model: DenseModel, max_rows: int = 16, packed: bool = True, kv_bits: int | None = None,
                 kv_group_size: int = 64):
        self.model = model
        self.engine = VerifyEngine(model, max_rows, packed=packed)
        self.max_rows = max_rows
        self.kv_bits, self.kv_group_size = kv_bits, kv_group_size

    def make_cache(self, capacity: int = 0) -> list:
        """The target's caches: quantized (mlx-lm QuantizedKVCache layout) when the target was
        built with ``kv_bits`` (target.py:166-184), plain bf16 otherwise."""
        return self.model.make_cache(capacity, self.kv_bits, self.kv_group_size)

    def _fused_rows(self, M: int, tap):
        """The step's tap output as the reference returns it: [1, M, n_tap * H], or None."""
        if tap is None:
            return None
        return self.engine.fused[:M].reshape(1, M, -1)

    def verify(self, ids: torch.Tensor, cache: list[KVCache], tap=None):
        """ids [1, 1+m] = [anchor] + m drafts -> (logits [1, 1+m, V], fused [1, 1+m, n_tap*H]),
        the residual stream after each tapped layer, in layer order (target.py:642-677,
        :208-220); ``tap=None`` skips the capture and returns ``fused=None``. Writes the rows
        into every layer's cache (offset advances by 1+m). Both results are views of the
        engine's buffers, valid until its next step."""
        flat = ids.reshape(-1)
        M = int(flat.numel())
        if not 1 <= M <= self.max_rows:
            raise ValueError(f"verify width {M} outside 1..{self.max_rows}")
        self.engine.set_tap(tap)
        for c in cache:
            c.reserve(M)
        pos0 = cache[0].offset
        self.engine.ids[:M].copy_(flat.to(self.engine.ids.device, torch.int64))
        logits = self.engine.step(M, cache, pos0)
        for c in cache:
            c.advance(M)
        return logits.reshape(1, M, -1), self._fused_rows(M, tap)

    def run(self, ids: torch.Tensor, cache: list[KVCache], tap):
        """ids [1, L] -> (logits [1, L, V], fused [1, L, n_tap*H] | None) through the module
        path (target.py:187-197 ``run``, the mlx-lm branch)."""
        hn, fused = self.model.body(ids.reshape(1, -1).to(self.model.embed_tokens.device, torch.int64), cache, tap)
        return self.model.lm_head(hn), fused

    def prefill(self, ids: torch.Tensor, cache: list[KVCache], tap=None, *, want_logits: bool = False,
                head_last_row: bool = True):
        """One prefill chunk -> ``(logits | None, fused | None)`` (target.py:435-465): the module
        path over ``ids`` [1, L] writing the caches, the tapped hidden states when ``tap`` is
        given, and the vocab projection only with ``want_logits`` (of the last row alone with
        ``head_last_row``). It runs under whatever projection scope is active;
        :func:`prefill_plain` chunks a prompt under the prefill wide path."""
        flat = ids.reshape(1, -1).to(self.model.embed_tokens.device, torch.int64)
        if flat.shape[1] == 0:
            raise ValueError("prefill: empty chunk")
        hn, fused = self.model.body(flat, cache, tap)
        if not want_logits:
            return None, fused
        return self.model.lm_head(hn[:, -1:] if head_last_row else hn), fused

    def rollback(self, cache: list[KVCache], n_rejected: int, accepted=None) -> None:
        """Dense rollback: trim every cache by the rejected rows; 0 is a no-op."""
        if n_rejected > 0:
            for c in cache:
                if c is not None and hasattr(c, "trim"):
                    c.trim(n_rejected)

    def greedy_round(self, pending: int, draft: list[int], cache: list[KVCache], tap=None):
        """One speculative round (generate.py:1544-1593): verify [pending] + draft, argmax and
        accept on the device, one host read, rollback of the rejected rows. Returns
        (n accepted drafts, committed tokens = accepted drafts + the target's bonus token,
        context rows): the context rows are ``fused[:, :n + 1]``, the tapped hidden states of
        [pending, accepted drafts] the drafter's ``update_context`` takes (generate.py:1590-1593),
        or None without a tap."""
        e = self.engine
        M = 1 + len(draft)
        if M > self.max_rows:
            raise ValueError(f"verify width {M} > {self.max_rows}")
        e.set_tap(tap)
        for c in cache:
            c.reserve(M)
        pos0 = cache[0].offset
        e.ids[:M].copy_(torch.tensor([pending] + list(draft), dtype=torch.int64))
        if draft:
            e.draft[:M - 1].copy_(torch.tensor(draft, dtype=torch.int32))
        e.step(M, cache, pos0, accept=True)
        for c in cache:
            c.advance(M)
        tt = e.tt[:M].tolist()                    # the round's one host read
        n = int(e.n_acc.item()) if draft else 0
        self.rollback(cache, len(draft) - n)
        fused = self._fused_rows(M, tap)
        return n, list(draft[:n]) + [int(tt[n])], None if fused is None else fused[:, :n + 1]


def prefill_plain(target: Target, ids: torch.Tensor, cache: list[KVCache], chunk: int | None = None,
                  tap=None):
    """Chunked prefill of a prompt before the verify loop (generate.py:1073-1100
    ``_prefill_plain``): pieces of at most ``chunk`` rows (default :data:`PREFILL_CHUNK`) under
    the prefill wide path the process has configured (``calibrate.apply_wide_gemm``,
    bit-identical to the stock path by its gate), the vocab projection of the last row of the
    last piece only. Returns (logits [1, 1, V], fused of the whole prompt | None)."""
    from . import calibrate
    from .wide_gemm import wide_matmul

    flat = ids.reshape(1, -1)
    L = int(flat.shape[1])
    if L == 0:
        raise ValueError("prefill: empty prompt")
    chunk = int(chunk or PREFILL_CHUNK)
    logits, pieces = None, []
    with wide_matmul(calibrate.WIDE_GEMM_MIN_ROWS, calibrate.WIDE_GEMM_SHAPES):
        for i in range(0, L, chunk):
            last = i + chunk >= L
            logits, fused = target.prefill(flat[:, i:i + chunk], cache, tap, want_logits=last, head_last_row=True)
            if fused is not None:
                pieces.append(fused)
    return logits, (torch.cat(pieces, dim=1) if pieces else None)


def greedy_generate(target: Target, prompt: list[int], steps: int) -> list[int]:
    """Plain greedy decoding (one token per forward): the reference output speculative
    decoding must reproduce."""
    cache = target.make_cache(len(prompt) + steps + 16)
    logits = None
    for i in range(0, len(prompt), target.max_rows):
        logits, _ = target.verify(torch.tensor([prompt[i:i + target.max_rows]]), cache)
    out = [int(torch.argmax(logits[0, -1].float()))]
    while len(out) < steps:
        logits, _ = target.verify(torch.tensor([[out[-1]]]), cache)
        out.append(int(torch.argmax(logits[0, -1].float())))
    return out
