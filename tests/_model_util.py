"""Shared helpers for the verify-forward tests: a tiny qwen3-style model and its numpy copy."""

from __future__ import annotations

import numpy as np
import torch

TINY = dict(hidden_size=256, num_hidden_layers=2, intermediate_size=512, num_attention_heads=4,
            num_key_value_heads=2, head_dim=128, vocab_size=512, rms_norm_eps=1e-6, rope_theta=1e6)


def tiny_model(device, seed=0, **kw):
    from dspark_rocm.model import DenseModel, ModelArgs

    return DenseModel.random(ModelArgs(**(TINY | kw)), device=device, seed=seed)


def _bf(t):
    return t.detach().float().cpu().numpy().astype(np.float32)


def _lin(l):
    return (l.weight.detach().cpu().numpy().view(np.uint32), _bf(l.scales), _bf(l.biases), l.bits)


def to_ref(model, matmul=None, embed=None, kv_bits=None):
    """The numpy oracle (oracle.model_ref.DenseRef) holding the same weights (``embed``: an
    object whose ``[ids]`` gives the embedding rows, instead of a copy of the whole table)."""
    from oracle.model_ref import DenseRef

    a = model.args
    layers = []
    for L in model.layers:
        at, mlp = L.self_attn, L.mlp
        layers.append(dict(input_norm=_bf(L.input_layernorm), post_norm=_bf(L.post_attention_layernorm),
                           q=_lin(at.q_proj), k=_lin(at.k_proj), v=_lin(at.v_proj), o=_lin(at.o_proj),
                           q_norm=_bf(at.q_norm), k_norm=_bf(at.k_norm),
                           gate=_lin(mlp.gate_proj), up=_lin(mlp.up_proj), down=_lin(mlp.down_proj)))
    cfg = dict(heads=a.num_attention_heads, kv_heads=a.num_key_value_heads, head_dim=a.head_dim,
               eps=a.rms_norm_eps, rope_theta=a.rope_theta)
    table = _bf(model.embed_tokens) if embed is None else embed
    return DenseRef(cfg, table, layers, _bf(model.norm), _lin(model.lm_head), matmul=matmul, kv_bits=kv_bits)
