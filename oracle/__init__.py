"""CPU oracle for the speculative-verify hot path — TEST INFRASTRUCTURE, not product code.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
anything from this package, and only to check results (or as the timed CPU baseline). The product
path (``mlx-dspark_amd``) never imports it.

What it restates (ARahim3/mlx-dspark v0.20.4, ``src/mlx_dspark/`` unless noted):

* :mod:`oracle.quant_ref` — the affine 4/8-bit packed format (skinny_qmm.py:95-119).
* :mod:`oracle.qmm_ref` — the factored small-M qmm (skinny_qmm.py:56-159, A.1).
* :mod:`oracle.attn_ref` — causal-in-block GQA verify attention: the exact definition
  (the fp32 SDPA the reference tests compare against, tests/test_multirow_attn.py:41-45) and a
  restatement of the multirow kernel's numerics (exp2 softmax, bf16 P, split-KV combine,
  multirow_attn.py:52-178); the row-split fallback (sdpa_split.py:61-93).
* :mod:`oracle.moe_ref` — softmax top-k routing and the grouped expert MLP (mlx-lm
  SparseMoeBlock / SwitchGLU, third-party; see its header).
* :mod:`oracle.verify_ref` — greedy accept and dense KV rollback (generate.py:1544-1593,
  target.py:679-696, batch_engine.py:220-224).
* ``dspark_oracle.c`` (built by ``oracle/Makefile`` into ``oracle/_build/liboracle.so``) —
  the same qmm / attention / routing in C with OpenMP, for large parity sizes and as the
  timed CPU baseline; loaded through :mod:`oracle.c_oracle`.

How each function is pinned (closed forms, brute force, invariants) is stated in its
docstring and exercised by ``tests/test_oracle_*.py``. The reference is Python + Metal and
cannot be built or imported here (mlx is not installed), so there is no ``oracle/_ref``.
"""
