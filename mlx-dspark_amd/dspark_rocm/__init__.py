"""dspark_rocm — MI355X (gfx950) speculative-verify hot path behind the reference's kernel calls.

Modules:
  _lib          ctypes binding of libdspark_rocm.so (C ABI: include/dspark.h)
  ops           torch-facing wrappers of every kernel entry point
  quant         the affine 4/8-bit packed format and a quantizer
  skinny_qmm    qmm / call / fits / plan (reference: skinny_qmm.py)
  small_m_qmm   QuantizedLinear routing scope (reference: small_m_qmm.py)
  multirow_attn multirow_sdpa / Window / MultirowConfig / scope (reference: multirow_attn.py)
  sdpa_split    row-split fallback scope (reference: sdpa_split.py)
  moe           routing, gather_qmm, SwitchGLU (reference: mlx-lm SparseMoeBlock / SwitchGLU)
  kv_cache      bf16 KV cache with O(1) trim (reference: BatchCache / mlx-lm KVCache)
"""

__version__ = "0.1.0"
