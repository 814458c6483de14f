"""Torch-facing wrappers of the C ABI: tensor checks, output allocation, current HIP stream.

These are the product path: every function here launches a hand-written gfx950 kernel through
``libdspark_rocm.so`` and raises if the library is unavailable or the call is refused.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

GROUP = 64


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("dspark kernels need tensors on a ROCm device (cuda:N)")


def _require_bf16(name: str, t: torch.Tensor) -> None:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name}: expected bfloat16, got {t.dtype}")


def _require_packed(w: torch.Tensor) -> None:
    if w.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"packed weights must be int32/uint32 words, got {w.dtype}")


def _rowmajor(name: str, t: torch.Tensor) -> None:
    if t.dim() != 2 or t.stride(-1) != 1:
        raise ValueError(f"{name}: expected a 2-D tensor with unit stride along the last dim")


# ---------------------------------------------------------------------------- quantized matmul


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                     *, group_size: int = GROUP, bits: int = 4, out: torch.Tensor | None = None
                     ) -> torch.Tensor:
    """``x [..., K] @ dequant(w)^T -> [..., N]`` (bf16) on the gfx950 qmm kernel.

    ``w`` packed [N, K*bits/32], ``scales``/``biases`` bf16 [N, K/64]. Any number of rows
    (served in 16-row tiles); the small-M shapes of speculative verify are the target.
    Mirrors ``mx.quantized_matmul(x, w, scales, biases, transpose=True, group_size, bits)``.
    """
    _require_cuda(x, w, scales, biases)
    _require_bf16("x", x)
    _require_packed(w)
    _require_bf16("scales", scales)
    _require_bf16("biases", biases)
    k = x.shape[-1]
    n = w.shape[0]
    if w.shape[1] * 32 // bits != k:
        raise ValueError(f"x K={k} does not match packed weight {tuple(w.shape)} at {bits} bits")
    if scales.shape != (n, k // group_size) or biases.shape != scales.shape:
        raise ValueError(f"scales/biases must be [{n}, {k // group_size}]")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    w = w.contiguous()
    scales = scales.contiguous()
    biases = biases.contiguous()
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    else:
        _rowmajor("out", out)
        if out.shape != (m, n) or out.dtype != torch.bfloat16:
            raise ValueError(f"out must be bf16 [{m}, {n}]")
    if m:
        nbytes = _lib.load().dspark_qmm_affine_workspace(m, k, n, bits, group_size)
        ws = qmm_workspace(x.device, nbytes)
        _lib.call("dspark_qmm_affine", _ptr(x2), x2.stride(0), m, k, _ptr(w), _ptr(scales),
                  _ptr(biases), n, bits, group_size, _ptr(out), out.stride(0), _ptr(ws),
                  0 if ws is None else ws.numel(), _stream(x))
    return out.reshape(*lead, n)


def quantized_matmul_multi(x_list, w_list, s_list, b_list, *, group_size: int = GROUP, bits: int = 4,
                           outs=None, workspace: torch.Tensor | None = None) -> list[torch.Tensor]:
    """Several ``quantized_matmul`` with the same M, K and bits in ONE launch (q/k/v; gate/up).
    The K slice count of a launch depends on the strips of all its problems, so a matrix gives
    the bits of a separate call whenever the launch keeps its slice count (the usual case; a
    different count reassociates the fp32 slice partials, within the qmm tolerance). An 8-bit
    [4096, 4096] matrix alone takes the whole-K kernel, which may also differ by an fp32 rounding
    of a bias term when one group of 64 x values spans many binades."""
    cnt = len(w_list)
    if not 1 <= cnt <= _lib.MAX_QMM_PROBLEMS:
        raise ValueError(f"1..{_lib.MAX_QMM_PROBLEMS} problems per launch, got {cnt}")
    if len(x_list) == 1 and cnt > 1:
        x_list = list(x_list) * cnt
    probs = (_lib.QmmProblem * cnt)()
    results = []
    m = None
    keep = []
    for i in range(cnt):
        x, w, s, b = x_list[i], w_list[i], s_list[i], b_list[i]
        _require_cuda(x, w, s, b)
        _require_bf16("x", x)
        _require_packed(w)
        k = x.shape[-1]
        x2 = x.reshape(-1, k)
        if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        if m is None:
            m = x2.shape[0]
        elif x2.shape[0] != m:
            raise ValueError("all problems must have the same number of rows")
        n = w.shape[0]
        w, s, b = w.contiguous(), s.contiguous(), b.contiguous()
        y = outs[i] if outs is not None else torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
        keep += [x2, w, s, b, y]
        probs[i] = _lib.QmmProblem(_ptr(x2), x2.stride(0), _ptr(w), _ptr(s), _ptr(b), _ptr(y), y.stride(0), n, k)
        results.append(y.reshape(*x.shape[:-1], n))
    nbytes = _lib.load().dspark_qmm_affine_multi_workspace(probs, cnt, m, bits, group_size)
    ws = _pick(workspace, x_list[0].device, nbytes, qmm=True)
    _lib.call("dspark_qmm_affine_multi", probs, cnt, m, bits, group_size, _ptr(ws),
              0 if ws is None else ws.numel(), _stream(x_list[0]))
    return results


class PackedQmm:
    """A quantized [N, K] matrix in the MI355X packed form (``dspark_qmm_pack``): 16-row weight
    tiles in the MFMA lane order plus 16-row x 8-group scale/bias tiles, in one uint8 buffer.
    Products equal those of the reference layout bit for bit."""

    def __init__(self, buf: torch.Tensor, n: int, k: int, bits: int):
        self.buf, self.n, self.k, self.bits = buf, n, k, bits

    @property
    def nbytes(self) -> int:
        return self.buf.numel()


def qmm_packable(n: int, k: int, bits: int, group_size: int = GROUP) -> bool:
    """True when ``dspark_qmm_pack`` accepts [n, k] (K % 512 == 0, 4/8-bit, groups of 64)."""
    return int(_lib.load().dspark_qmm_packed_bytes(n, k, bits, group_size)) > 0


def qmm_pack(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *, bits: int,
             group_size: int = GROUP) -> PackedQmm:
    """Pack the reference layout (uint32 [N, K*bits/32], bf16 scales/biases [N, K/64]) once."""
    _require_cuda(w, scales, biases)
    _require_packed(w)
    n, k = w.shape[0], w.shape[1] * 32 // bits
    w, scales, biases = w.contiguous(), scales.contiguous(), biases.contiguous()
    lib = _lib.load()
    nbytes = int(lib.dspark_qmm_packed_bytes(n, k, bits, group_size))
    if nbytes == 0:
        raise _lib.DsparkError("dspark_qmm_pack", -2, f"[{n}, {k}] {bits}-bit cannot be packed (K % 512 != 0)")
    buf = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
    _lib.call("dspark_qmm_pack", _ptr(w), _ptr(scales), _ptr(biases), n, k, bits, group_size, _ptr(buf), nbytes,
              _stream(w))
    return PackedQmm(buf, n, k, bits)


def _packed_problems(x_list, packed_list, outs):
    """(problems, count, M, bits, results, keep-alive list) of a packed multi launch. One x
    tensor given for several problems stays one x (one copy when it must be made contiguous),
    which the one-workgroup-per-CU kernel requires."""
    cnt = len(packed_list)
    if not 1 <= cnt <= _lib.MAX_QMM_PROBLEMS:
        raise ValueError(f"1..{_lib.MAX_QMM_PROBLEMS} problems per launch, got {cnt}")
    if len(x_list) == 1 and cnt > 1:
        x_list = list(x_list) * cnt
    bits = packed_list[0].bits
    probs = (_lib.QmmPackedProblem * cnt)()
    results, keep, m, rows = [], [], None, {}
    for i in range(cnt):
        x, pq = x_list[i], packed_list[i]
        _require_cuda(x, pq.buf)
        _require_bf16("x", x)
        if pq.bits != bits:
            raise ValueError("all packed problems of one launch must share bits")
        k = x.shape[-1]
        if k != pq.k:
            raise ValueError(f"x has K={k}, the packed matrix K={pq.k}")
        x2 = rows.get(id(x))
        if x2 is None:
            x2 = x.reshape(-1, k)
            if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
                x2 = x2.contiguous()
            rows[id(x)] = x2
        if m is None:
            m = x2.shape[0]
        elif x2.shape[0] != m:
            raise ValueError("all problems must have the same number of rows")
        y = outs[i] if outs is not None else torch.empty((m, pq.n), dtype=torch.bfloat16, device=x.device)
        keep += [x, x2, y]
        probs[i] = _lib.QmmPackedProblem(_ptr(x2), x2.stride(0), _ptr(pq.buf), _ptr(y), y.stride(0), pq.n, k)
        results.append(y.reshape(*x.shape[:-1], pq.n))
    return probs, cnt, m, bits, results, keep


PACKED_KERNELS = ("split-K", "whole-K tile", "per CU")


def packed_multi_plan(x_list, packed_list, *, group_size: int = GROUP) -> dict:
    """The kernel ``quantized_matmul_packed_multi`` runs for these operands (host-only query):
    ``kernel`` (one of ``PACKED_KERNELS``), ``slices`` (the split-K association the bits
    follow), ``tiles_per_workgroup`` and ``k_parts`` (per-CU kernel: workgroups per row tile
    along K) and ``workgroups``."""
    probs, cnt, m, bits, _, keep = _packed_problems(x_list, packed_list, None)
    out = (ctypes.c_int32 * 5)()
    _lib.call("dspark_qmm_packed_multi_plan", probs, cnt, m, bits, group_size, out)
    return {"kernel": PACKED_KERNELS[out[0]], "slices": out[1], "tiles_per_workgroup": out[2],
            "workgroups": out[3], "k_parts": out[4]}


def quantized_matmul_packed_multi(x_list, packed_list, *, group_size: int = GROUP, outs=None,
                                  workspace: torch.Tensor | None = None) -> list[torch.Tensor]:
    """``quantized_matmul_multi`` over packed matrices (one launch, same M, K and bits)."""
    probs, cnt, m, bits, results, keep = _packed_problems(x_list, packed_list, outs)
    nbytes = _lib.load().dspark_qmm_packed_multi_workspace(probs, cnt, m, bits, group_size)
    ws = _pick(workspace, x_list[0].device, nbytes, qmm=True)
    _lib.call("dspark_qmm_packed_multi", probs, cnt, m, bits, group_size, _ptr(ws),
              0 if ws is None else ws.numel(), _stream(x_list[0]))
    return results


def quantized_matmul_packed(x: torch.Tensor, packed: PackedQmm, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """``x [.., K] @ dequant(W)^T`` for a packed W -> ``[.., N]`` bf16."""
    return quantized_matmul_packed_multi([x], [packed], outs=None if out is None else [out])[0]


class PackedSwiGLU:
    """Gate and up [N, K] matrices in the pair form (``dspark_qmm_pack_swiglu``): the packed
    layout of 2 ceil(N/16) row tiles, gate tile t then up tile t, for the fused gate / up /
    SwiGLU launch."""

    def __init__(self, buf: torch.Tensor, n: int, k: int, bits: int):
        self.buf, self.n, self.k, self.bits = buf, n, k, bits


def qmm_pack_swiglu(gate, up, *, bits: int, group_size: int = GROUP) -> PackedSwiGLU:
    """Pack (w, scales, biases) of the gate and of the up projection (same shape) into the pair
    form once."""
    (gw, gs, gb), (uw, us, ub) = gate, up
    _require_cuda(gw, gs, gb, uw, us, ub)
    _require_packed(gw)
    _require_packed(uw)
    if gw.shape != uw.shape or gs.shape != us.shape:
        raise ValueError(f"gate {tuple(gw.shape)} and up {tuple(uw.shape)} must have one shape")
    n, k = gw.shape[0], gw.shape[1] * 32 // bits
    args = [t.contiguous() for t in (gw, gs, gb, uw, us, ub)]
    lib = _lib.load()
    nbytes = int(lib.dspark_qmm_swiglu_packed_bytes(n, k, bits, group_size))
    if nbytes == 0:
        raise _lib.DsparkError("dspark_qmm_pack_swiglu", -2, f"[{n}, {k}] {bits}-bit cannot be packed (K % 512 != 0)")
    buf = torch.empty(nbytes, dtype=torch.uint8, device=gw.device)
    _lib.call("dspark_qmm_pack_swiglu", *[_ptr(t) for t in args], n, k, bits, group_size, _ptr(buf), nbytes,
              _stream(gw))
    return PackedSwiGLU(buf, n, k, bits)


def quantized_swiglu_packed(x: torch.Tensor, pair: PackedSwiGLU, *, group_size: int = GROUP,
                            out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(x W_gate^T) * (x W_up^T)`` with mlx's bf16 rounding, in one launch -> ``[.., N]``."""
    _require_cuda(x, pair.buf)
    _require_bf16("x", x)
    k = x.shape[-1]
    if k != pair.k:
        raise ValueError(f"x has K={k}, the packed pair K={pair.k}")
    x2 = x.reshape(-1, k)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    h = out if out is not None else torch.empty((m, pair.n), dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    nbytes = lib.dspark_qmm_swiglu_packed_workspace(pair.n, k, m, pair.bits, group_size)
    ws = _pick(workspace, x.device, nbytes, qmm=True)
    _lib.call("dspark_qmm_swiglu_packed", _ptr(x2), x2.stride(0), _ptr(pair.buf), _ptr(h), h.stride(0), pair.n, k, m,
              pair.bits, group_size, _ptr(ws), 0 if ws is None else ws.numel(), _stream(x))
    return h.reshape(*x.shape[:-1], pair.n)


DEQUANT_DTYPES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}   # dspark_dtype codes


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *, bits: int,
               group_size: int = GROUP, dtype: torch.dtype = torch.float32,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """Packed affine ``w [N, K*bits/32]`` -> ``[N, K]`` in ``dtype`` in one launch
    (``dspark_qmm_dequantize``): ``(scale * q) + bias`` as an fp32 product rounded, then an fp32
    sum rounded, then rounded to ``dtype``; for fp32 these are the bits of
    :func:`dspark_rocm.quant.dequantize` (the reference's ``mx.dequantize``, wide_gemm.py:222)."""
    _require_cuda(w, scales, biases)
    _require_packed(w)
    _rowmajor("w", w)
    if scales.dtype not in DEQUANT_DTYPES or biases.dtype != scales.dtype or dtype not in DEQUANT_DTYPES:
        raise TypeError(f"dequantize: scales/biases {scales.dtype}/{biases.dtype}, out {dtype}")
    n, k = int(w.shape[0]), int(w.shape[1]) * 32 // bits
    scales, biases = scales.contiguous(), biases.contiguous()
    if out is None:
        out = torch.empty((n, k), dtype=dtype, device=w.device)
    elif out.dtype != dtype or tuple(out.shape) != (n, k) or out.stride(-1) != 1:
        raise ValueError(f"dequantize: out must be [{n}, {k}] {dtype} with unit inner stride")
    _lib.call("dspark_qmm_dequantize", _ptr(w), _ptr(scales), _ptr(biases), DEQUANT_DTYPES[scales.dtype], n, k,
              bits, group_size, DEQUANT_DTYPES[dtype], _ptr(out), out.stride(0), _stream(out))
    return out


def stream_read(buf: torch.Tensor, sink: torch.Tensor) -> None:
    """Read every byte of ``buf`` once on the gfx950 streaming-read probe (``dspark_stream_read``);
    ``sink`` is an int32 scalar tensor the kernel practically never writes. For timing."""
    _require_cuda(buf, sink)
    if not buf.is_contiguous():
        raise ValueError("stream_read: contiguous buffer")
    _lib.call("dspark_stream_read", _ptr(buf), buf.numel() * buf.element_size(), _ptr(sink), _stream(buf))


def qmm_supported(m: int, k: int, n: int, bits: int, group_size: int = GROUP) -> bool:
    return _lib.load().dspark_qmm_affine_supported(m, k, n, bits, group_size) == 0


# ---------------------------------------------------------------------------- workspaces

_workspaces: dict[tuple[int, int], torch.Tensor] = {}
_qmm_workspaces: dict[tuple[int, int], torch.Tensor] = {}
# Buffers a larger request superseded. They are never freed: a HIP graph captured earlier may
# still hold their addresses, and freeing one would let the caching allocator hand that memory
# to another tensor which the next replay then overwrites.
_retired: list[torch.Tensor] = []


def _stream_key(device) -> tuple[torch.device, tuple[int, int]]:
    dev = torch.device(device)
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    return dev, (idx, torch.cuda.current_stream(dev).cuda_stream)


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A per-(device, stream) scratch buffer reused across calls (stream-ordered reuse is safe;
    two streams never share one). Grows by replacement; a replaced buffer stays allocated."""
    if nbytes <= 0:
        return None
    dev, key = _stream_key(device)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _retired.append(buf)
        buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
        _workspaces[key] = buf
    return buf


def qmm_workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """The qmm workspace of (device, current stream): zero-filled when allocated (its arrival
    counters must start at zero; every qmm call leaves them zero). Kept apart from the other
    scratch buffers, which hold arbitrary data between calls. A replaced buffer stays
    allocated, as for :func:`workspace`."""
    if nbytes <= 0:
        return None
    dev, key = _stream_key(device)
    buf = _qmm_workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _retired.append(buf)
        buf = torch.zeros(max(nbytes, 4 << 20), dtype=torch.uint8, device=dev)
        _qmm_workspaces[key] = buf
    return buf


def new_qmm_workspace(device, nbytes: int) -> torch.Tensor | None:
    """A caller-owned qmm workspace of at least ``nbytes`` (zeroed: the arrival counters must
    start at zero), e.g. for a graph-captured engine that must not share the per-stream one."""
    if nbytes <= 0:
        return None
    return torch.zeros(max(int(nbytes), 256 << 10), dtype=torch.uint8, device=device)


def qmm_launch_workspace_bytes(m: int, k: int, ns, bits: int, group_size: int = GROUP) -> int:
    """Workspace bytes of one qmm launch over matrices [n, k] for n in ``ns`` with ``m`` rows
    (the reference and the packed layout plan alike). Host query only: the problem pointers it
    passes are placeholders the library does not dereference."""
    ns = list(ns)
    probs = (_lib.QmmProblem * len(ns))()
    for i, n in enumerate(ns):
        probs[i] = _lib.QmmProblem(256, k, 256, 256, 256, 256, n, n, k)
    return int(_lib.load().dspark_qmm_affine_multi_workspace(probs, len(ns), m, bits, group_size))


def attention_workspace_bound(batch: int, hq: int, hk: int, d: int, max_rows: int) -> int:
    """The most workspace bytes verify attention needs for up to ``max_rows`` query rows at any
    cache length: the plan caps its key blocks by the grid size, not by the length."""
    lib = _lib.load()
    return max(int(lib.dspark_verify_attention_workspace(batch, hq, hk, m, d, 1 << 29)) for m in range(1, max_rows + 1))


def qmm_workspace_reset(ws: torch.Tensor) -> None:
    """Zero the split-K arrival counters of a qmm workspace on the current stream (a fill
    kernel, so it may be captured): restores the state every completed qmm call leaves."""
    _require_cuda(ws)
    _lib.call("dspark_qmm_workspace_reset", _ptr(ws), ws.numel(), _stream(ws))


def _pick(ws: torch.Tensor | None, device, nbytes: int, qmm: bool):
    """The caller's workspace when given (checked for size), else the per-stream one."""
    if ws is None:
        return qmm_workspace(device, nbytes) if qmm else workspace(device, nbytes)
    if ws.numel() < nbytes:
        raise ValueError(f"workspace of {ws.numel()} bytes < {nbytes} needed")
    return ws


# ---------------------------------------------------------------------------- verify attention

ATTN_HEAD_DIMS = (64, 128, 256)   # kernel instances; any head dim d % 8 == 0, d <= 256 runs on the next one up
QUANT_HEAD_DIMS = (64, 128, 256)  # quantized caches: whole groups of 64 along the head dim


def attn_head_dim_ok(d: int) -> bool:
    """The reference's head-dim rule (multirow_attn.py:200, :306): d % 8 == 0 and d <= 256."""
    return 8 <= d <= 256 and d % 8 == 0
ATTN_DTYPES = {torch.bfloat16: 0, torch.float16: 1}   # dspark_dtype codes
KV_BITS = (4, 8)


def _i64x3(t: torch.Tensor):
    arr = (ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2))
    return arr


def _attn_dtype(q: torch.Tensor, *others: torch.Tensor) -> int:
    if q.dtype not in ATTN_DTYPES:
        raise TypeError(f"verify attention: q dtype {q.dtype} (bfloat16 or float16)")
    for t in others:
        if t.dtype != q.dtype:
            raise TypeError(f"verify attention: {t.dtype} does not match q's {q.dtype}")
    return ATTN_DTYPES[q.dtype]


def _attn_shapes(q, k, v):
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dim() != 4:
            raise ValueError(f"{name}: expected [B, H, L, D]")
    B, Hq, mq, D = q.shape
    Hk, L = k.shape[1], k.shape[2]
    if k.shape != (B, Hk, L, D) or v.shape != (B, Hk, L, D):
        raise ValueError(f"k/v must be [{B}, Hk, L, {D}]; got {tuple(k.shape)} / {tuple(v.shape)}")
    if k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("k/v must be contiguous along head_dim")
    return B, Hq, mq, D, Hk, L


def verify_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float, causal: bool = True,
                     tree_anc: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``softmax(scale * q k^T + mask) v`` for few verify rows over a (strided) KV cache view.

    q bf16 or fp16 [B, Hq, Mq, D] (D % 8 == 0, D <= 256); k/v of q's dtype [B, Hk, L, D] with unit
    stride along D (any batch/head/seq strides, e.g. a ``[..., :L, :]`` slice of a larger
    cache). ``causal``: row i sees keys ``0 .. L - Mq + i``. ``tree_anc`` (uint32/int32 [Mq])
    selects the tree-verify mask.
    """
    _require_cuda(q, k, v)
    dt = _attn_dtype(q, k, v)
    B, Hq, mq, D, Hk, L = _attn_shapes(q, k, v)
    q = q.contiguous()
    if out is None:
        out = torch.empty_like(q)
    osr = (ctypes.c_int64 * 3)(Hq * mq * D, mq * D, D)
    return _launch_attention(dt, q, k, v, out, osr, scale, causal, tree_anc, None)


def _launch_attention(dt, q, k, v, out, out_strides, scale, causal, tree_anc, ws):
    B, Hq, mq, D = q.shape
    Hk, L = k.shape[1], k.shape[2]
    nbytes = _lib.load().dspark_verify_attention_workspace(B, Hq, Hk, mq, D, L)
    ws = _pick(ws, q.device, nbytes, qmm=False)
    anc = None if tree_anc is None else tree_anc.to(device=q.device, dtype=torch.int32).contiguous()
    _lib.call("dspark_verify_attention_typed", dt, _ptr(q), B, Hq, mq, D, _ptr(k), _ptr(v), _i64x3(k), _i64x3(v),
              Hk, L, float(scale), int(bool(causal)), _ptr(anc), _ptr(out), out_strides, _ptr(ws),
              0 if ws is None else ws.numel(), _stream(q))
    return out


def verify_attention_blocks(B: int, Hq: int, Hk: int, mq: int, D: int, L: int) -> int:
    return int(_lib.load().dspark_verify_attention_blocks(B, Hq, Hk, mq, D, L))


def verify_attention_quantized(q: torch.Tensor, keys, values, *, scale: float, causal: bool = True, bits: int = 8,
                               group_size: int = GROUP, out: torch.Tensor | None = None, out_strides=None,
                               workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Verify attention over a quantized KV cache (mlx-lm ``QuantizedKVCache`` state).

    ``keys`` / ``values`` = (words int32 [B, Hk, L, D*bits/32], scales [B, Hk, L, D/64],
    biases [B, Hk, L, D/64]) with scales/biases in q's dtype, fields of ``bits`` (4 or 8)
    along D, low bits first; any batch/head/seq strides (cache views), unit stride along the
    last dim. Semantics: attention over ``scale * q_field + bias`` per group of 64 values.
    ``out_strides`` = (batch, query head, position) element strides of ``out`` (head_dim
    contiguous), e.g. [B, Mq, Hq*D] rows for o_proj; default a contiguous [B, Hq, Mq, D].
    """
    kw, ks, kb = keys
    vw, vs, vb = values
    _require_cuda(q, kw, ks, kb, vw, vs, vb)
    dt = _attn_dtype(q, ks, kb, vs, vb)
    if bits not in KV_BITS:
        raise ValueError(f"bits={bits} (4 or 8)")
    for t in (kw, vw):
        _require_packed(t)
    B, Hq, mq, D = q.shape
    if D not in QUANT_HEAD_DIMS:
        raise ValueError(f"quantized caches: head_dim {D} (64, 128 or 256)")
    Hk, L = kw.shape[1], kw.shape[2]
    W, G = D * bits // 32, D // group_size
    for name, t, last in (("key words", kw, W), ("value words", vw, W), ("key scales", ks, G), ("key biases", kb, G),
                          ("value scales", vs, G), ("value biases", vb, G)):
        if t.dim() != 4 or tuple(t.shape) != (B, Hk, L, last) or t.stride(-1) != 1:
            raise ValueError(f"{name}: expected [{B}, {Hk}, {L}, {last}] with unit last stride, got {tuple(t.shape)}")
    if ks.stride() != kb.stride() or vs.stride() != vb.stride():
        raise ValueError("scales and biases of one cache must share strides")
    q = q.contiguous()
    if out is None:
        if out_strides is not None:
            raise ValueError("out_strides needs out")
        out = torch.empty_like(q)
    if out.dtype != q.dtype:
        raise TypeError(f"out dtype {out.dtype} does not match q's {q.dtype}")
    osr = (ctypes.c_int64 * 3)(*([Hq * mq * D, mq * D, D] if out_strides is None else [int(x) for x in out_strides]))
    nbytes = _lib.load().dspark_verify_attention_workspace(B, Hq, Hk, mq, D, L)
    ws = _pick(workspace, q.device, nbytes, qmm=False)
    _lib.call("dspark_verify_attention_quantized", dt, _ptr(q), B, Hq, mq, D, _ptr(kw), _ptr(ks), _ptr(kb), _i64x3(kw),
              _i64x3(ks), _ptr(vw), _ptr(vs), _ptr(vb), _i64x3(vw), _i64x3(vs), Hk, L, float(scale),
              int(bool(causal)), bits, group_size, _ptr(out), osr, _ptr(ws), 0 if ws is None else ws.numel(),
              _stream(q))
    return out


# ---------------------------------------------------------------------------- MoE

def moe_route(logits: torch.Tensor, k: int, *, renorm: bool = True, bucket: bool = False):
    """Softmax top-k routing on the GPU. logits bf16 [M, E] -> (inds int32 [M, k], scores bf16
    [M, k]) and, with ``bucket=True``, also (expert_offsets [E+1], sorted_pairs [M*k],
    pair_pos [M*k]) of the (token, slot) pairs sorted by expert."""
    _require_cuda(logits)
    _require_bf16("logits", logits)
    logits = logits.contiguous()
    M, E = logits.shape
    dev = logits.device
    inds = torch.empty((M, k), dtype=torch.int32, device=dev)
    scores = torch.empty((M, k), dtype=torch.bfloat16, device=dev)
    off = srt = pos = None
    if bucket:
        off = torch.empty(E + 1, dtype=torch.int32, device=dev)
        srt = torch.empty(M * k, dtype=torch.int32, device=dev)
        pos = torch.empty(M * k, dtype=torch.int32, device=dev)
    _lib.call("dspark_moe_route_topk", _ptr(logits), M, E, k, int(bool(renorm)), _ptr(inds), _ptr(scores),
              _ptr(off), _ptr(srt), _ptr(pos), _stream(logits))
    if bucket:
        return inds, scores, off, srt, pos
    return inds, scores


def gather_qmm_sorted(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                      expert_offsets: torch.Tensor, *, row_index: torch.Tensor | None = None, bits: int = 4,
                      group_size: int = GROUP, rows: int | None = None) -> torch.Tensor:
    """Grouped qmm over expert-sorted rows: ``y[p] = x[row_index[p]] @ dequant(w[e])^T`` for
    ``expert_offsets[e] <= p < expert_offsets[e+1]``. w packed [E, N, K*bits/32]."""
    _require_cuda(x, w, scales, biases, expert_offsets)
    _require_bf16("x", x)
    _require_packed(w)
    E, N = w.shape[0], w.shape[1]
    K = x.shape[-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    P = rows if rows is not None else (row_index.numel() if row_index is not None else x2.shape[0])
    y = torch.empty((P, N), dtype=torch.bfloat16, device=x.device)
    ri = None if row_index is None else row_index.to(torch.int32).contiguous()
    _lib.call("dspark_gather_qmm", _ptr(x2), x2.stride(0), K, _ptr(ri), _ptr(expert_offsets.to(torch.int32).contiguous()),
              E, P, _ptr(w.contiguous()), _ptr(scales.contiguous()), _ptr(biases.contiguous()), N, bits, group_size,
              _ptr(y), y.stride(0), _stream(x))
    return y


class PackedExperts:
    """Stacked expert weights [E, N, K*bits/32] in the packed form of ``dspark_moe_pack``: each
    expert's 16-row tiles in the MFMA lane order (the same bytes; scales and biases are not part
    of it and keep their [E, N, K/64] layout)."""

    def __init__(self, buf: torch.Tensor, experts: int, n: int, k: int, bits: int):
        self.buf, self.experts, self.n, self.k, self.bits = buf, experts, n, k, bits


def moe_packable(experts: int, n: int, k: int, bits: int, group_size: int = GROUP) -> bool:
    return int(_lib.load().dspark_moe_packed_bytes(experts, n, k, bits, group_size)) > 0


MOE_KERNELS = ("expert x strip", "per CU")


def moe_packed_plan(M: int, H: int, I: int, E: int, k: int, bits: int) -> dict:
    """The expert kernels ``moe_switch_glu`` runs over packed experts for this shape (host-only
    query): ``gate_up`` and ``down``, each one of ``MOE_KERNELS``."""
    out = (ctypes.c_int32 * 2)()
    _lib.call("dspark_moe_packed_plan", M, H, I, E, k, bits, out)
    return {"gate_up": MOE_KERNELS[out[0]], "down": MOE_KERNELS[out[1]]}


def moe_pack(w: torch.Tensor, *, bits: int, group_size: int = GROUP) -> PackedExperts:
    """Pack stacked expert weights (int32 [E, N, K*bits/32]) once (N % 16 == 0, K % 128 == 0)."""
    _require_cuda(w)
    _require_packed(w)
    E, n, k = w.shape[0], w.shape[1], w.shape[2] * 32 // bits
    w = w.contiguous()
    nbytes = int(_lib.load().dspark_moe_packed_bytes(E, n, k, bits, group_size))
    if nbytes == 0:
        raise _lib.DsparkError("dspark_moe_pack", -2, f"[{E}, {n}, {k}] {bits}-bit cannot be packed "
                                                      "(N % 16 == 0 and K % 128 == 0 needed)")
    buf = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
    _lib.call("dspark_moe_pack", _ptr(w), E, n, k, bits, group_size, _ptr(buf), nbytes, _stream(w))
    return PackedExperts(buf, E, n, k, bits)


def moe_switch_glu(x: torch.Tensor, logits: torch.Tensor, gate, up, down, *, k: int, bits: int = 4,
                   renorm: bool = True, group_size: int = GROUP):
    """Routed-expert SwiGLU MLP of one MoE block: route -> gate/up (fused SwiGLU) -> down ->
    score-weighted combine, four launches. ``gate``/``up``/``down`` are (w, scales, biases) with
    w int32 [E, rows, cols*bits/32], or a :class:`PackedExperts` of it (``dspark_moe_switch_glu_packed``,
    the same results bit for bit). Returns (out bf16 [M, H], inds [M, k], scores [M, k])."""
    _require_cuda(x, logits)
    _require_bf16("x", x)
    _require_bf16("logits", logits)
    x = x.contiguous()
    logits = logits.contiguous()
    M, H = x.shape
    E = logits.shape[1]
    packed = isinstance(gate[0], PackedExperts)
    if packed != isinstance(up[0], PackedExperts) or packed != isinstance(down[0], PackedExperts):
        raise ValueError("moe_switch_glu: gate, up and down must all be packed or all row-major")
    I = gate[0].n if packed else gate[0].shape[1]
    lib = _lib.load()
    nbytes = lib.dspark_moe_workspace(M, H, I, E, k)
    if nbytes == 0:
        raise ValueError(f"unsupported MoE shape M={M} E={E} k={k}")
    ws = workspace(x.device, nbytes)
    out = torch.empty((M, H), dtype=torch.bfloat16, device=x.device)
    inds = torch.empty((M, k), dtype=torch.int32, device=x.device)
    scores = torch.empty((M, k), dtype=torch.bfloat16, device=x.device)
    (wg, sg, bg), (wu, su, bu), (wd, sd, bd) = gate, up, down
    if packed:
        wg, wu, wd = wg.buf, wu.buf, wd.buf
    _lib.call("dspark_moe_switch_glu_packed" if packed else "dspark_moe_switch_glu", _ptr(x), _ptr(logits), M, H, I,
              E, k, int(bool(renorm)), _ptr(wg), _ptr(sg), _ptr(bg), _ptr(wu), _ptr(su), _ptr(bu), _ptr(wd),
              _ptr(sd), _ptr(bd), bits, group_size, _ptr(out), _ptr(inds), _ptr(scores), _ptr(ws), ws.numel(),
              _stream(x))
    return out, inds, scores


def verify_attention_into(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor, out_strides, *,
                          scale: float, causal: bool = True, tree_anc: torch.Tensor | None = None,
                          workspace: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`verify_attention` writing through element strides ``out_strides`` = (batch, query
    head, position) of ``out`` (head_dim contiguous), e.g. [B, Mq, Hq*D] rows for o_proj."""
    _require_cuda(q, k, v, out)
    dt = _attn_dtype(q, k, v, out)
    _attn_shapes(q, k, v)
    q = q.contiguous()
    osr = (ctypes.c_int64 * 3)(*[int(x) for x in out_strides])
    return _launch_attention(dt, q, k, v, out, osr, scale, causal, tree_anc, workspace)


# ---------------------------------------------------------------------------- verify-forward layer ops

def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, *, residual: torch.Tensor | None = None,
            h_out: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``bf16(bf16(h * rsqrt(mean(h^2) + eps)) * w)`` per row, h = x or bf16(x + residual)
    (written to ``h_out`` when given). x [M, H] bf16."""
    _require_cuda(x, w)
    _require_bf16("x", x)
    M, H = x.shape
    if out is None:
        out = torch.empty((M, H), dtype=torch.bfloat16, device=x.device)
    _lib.call("dspark_rmsnorm", _ptr(x), x.stride(0), _ptr(residual), 0 if residual is None else residual.stride(0),
              _ptr(w), M, H, float(eps), _ptr(h_out), 0 if h_out is None else h_out.stride(0), _ptr(out),
              out.stride(0), _stream(x))
    return out


def qk_norm_rope_kv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_norm_w: torch.Tensor,
                    k_norm_w: torch.Tensor, *, heads: int, kv_heads: int, head_dim: int, eps: float,
                    rope_base: float, pos0: int, q_out: torch.Tensor, k_cache: torch.Tensor,
                    v_cache: torch.Tensor) -> torch.Tensor:
    """q/k RMSNorm + RoPE at positions pos0.. and the cache write. q [M, Hq*D], k/v [M, Hk*D];
    q_out [Hq, M, D]; k_cache/v_cache [Hk, capacity, D] views (batch 1)."""
    _require_cuda(q, k, v, q_out, k_cache, v_cache)
    M = q.shape[0]
    if k_cache.shape[1] < pos0 + M or v_cache.shape[1] < pos0 + M:
        raise ValueError(f"cache capacity {k_cache.shape[1]} < pos0 + M = {pos0 + M}")
    ks = (ctypes.c_int64 * 2)(k_cache.stride(0), k_cache.stride(1))
    vs = (ctypes.c_int64 * 2)(v_cache.stride(0), v_cache.stride(1))
    _lib.call("dspark_qk_norm_rope_kv", _ptr(q), q.stride(0), _ptr(k), k.stride(0), _ptr(v), v.stride(0), M, heads,
              kv_heads, head_dim, _ptr(q_norm_w), _ptr(k_norm_w), float(eps), float(rope_base), int(pos0),
              _ptr(q_out), _ptr(k_cache), ks, _ptr(v_cache), vs, _stream(q))
    return q_out


def qk_norm_rope_kv_quantized(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_norm_w: torch.Tensor,
                              k_norm_w: torch.Tensor, *, heads: int, kv_heads: int, head_dim: int, eps: float,
                              rope_base: float, pos0: int, q_out: torch.Tensor, k_cache, v_cache, bits: int,
                              group_size: int = GROUP) -> torch.Tensor:
    """:func:`qk_norm_rope_kv` into a quantized cache: ``k_cache`` / ``v_cache`` are the
    (words [Hk, capacity, D*bits/32], scales [Hk, capacity, D/64], biases) triples of one
    layer (batch 1, bf16 scales); the rows at pos0.. are quantized as ``quant.quantize_rows``
    quantizes the values the plain kernel would write."""
    kw, ks, kb = k_cache
    vw, vs, vb = v_cache
    _require_cuda(q, k, v, q_out, kw, ks, kb, vw, vs, vb)
    for t in (ks, kb, vs, vb):
        _require_bf16("cache scales / biases", t)
    M = q.shape[0]
    for name, t in (("key words", kw), ("value words", vw), ("key scales", ks), ("value scales", vs)):
        if t.dim() != 3 or t.shape[1] < pos0 + M or t.stride(-1) != 1:
            raise ValueError(f"{name}: expected [Hk, capacity >= {pos0 + M}, ...] with unit last stride")
    if ks.stride() != kb.stride() or vs.stride() != vb.stride():
        raise ValueError("scales and biases of one cache must share strides")
    two = lambda t: (ctypes.c_int64 * 2)(t.stride(0), t.stride(1))
    _lib.call("dspark_qk_norm_rope_kv_quantized", _ptr(q), q.stride(0), _ptr(k), k.stride(0), _ptr(v), v.stride(0), M,
              heads, kv_heads, head_dim, _ptr(q_norm_w), _ptr(k_norm_w), float(eps), float(rope_base), int(pos0),
              _ptr(q_out), _ptr(kw), _ptr(ks), _ptr(kb), two(kw), two(ks), _ptr(vw), _ptr(vs), _ptr(vb), two(vw),
              two(vs), int(bits), int(group_size), _stream(q))
    return q_out


def swiglu(g: torch.Tensor, u: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``bf16(bf16(g * bf16(sigmoid(g))) * u)`` (mlx's silu(g) * u)."""
    _require_cuda(g, u)
    M, N = g.shape
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=g.device)
    _lib.call("dspark_swiglu", _ptr(g), g.stride(0), _ptr(u), u.stride(0), M, N, _ptr(out), out.stride(0), _stream(g))
    return out


def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """int32 [M]: first index of each row's maximum (bf16 logits [M, V])."""
    _require_cuda(logits)
    _require_bf16("logits", logits)
    M, V = logits.shape
    if out is None:
        out = torch.empty(M, dtype=torch.int32, device=logits.device)
    _lib.call("dspark_argmax_rows", _ptr(logits), logits.stride(0), M, V, _ptr(out), _stream(logits))
    return out


def greedy_accept(draft: torch.Tensor, target_tokens: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """int32 [1]: length of the accepted draft prefix (draft == target_tokens[:m] while equal)."""
    _require_cuda(target_tokens)
    m = int(draft.numel())
    if out is None:
        out = torch.empty(1, dtype=torch.int32, device=target_tokens.device)
    d = draft.to(device=target_tokens.device, dtype=torch.int32).contiguous() if m else None
    _lib.call("dspark_greedy_accept", _ptr(d), m, _ptr(target_tokens), _ptr(out), _stream(target_tokens))
    return out


def argmax_accept_workspace_bytes(M: int, V: int) -> int:
    """Workspace bytes of :func:`argmax_accept` for ``M`` rows of ``V`` logits."""
    return int(_lib.load().dspark_argmax_accept_workspace(M, V))


def argmax_accept(logits: torch.Tensor, draft: torch.Tensor, target_tokens: torch.Tensor, n_accepted: torch.Tensor,
                  workspace: torch.Tensor) -> None:
    """:func:`argmax_rows` into ``target_tokens`` and :func:`greedy_accept` of ``draft`` into
    ``n_accepted``, in one launch. ``workspace`` (uint8, >= :func:`argmax_accept_workspace_bytes`,
    zero-filled when allocated) holds an arrival counter that every call leaves at zero."""
    _require_cuda(logits, target_tokens, n_accepted, workspace)
    _require_bf16("logits", logits)
    M, V = logits.shape
    m = int(draft.numel())
    if m and (draft.dtype != torch.int32 or not draft.is_contiguous() or draft.device != logits.device):
        raise ValueError("argmax_accept: draft must be a contiguous int32 tensor on the logits' device")
    _lib.call("dspark_argmax_accept", _ptr(logits), logits.stride(0), M, V, _ptr(draft) if m else None, m,
              _ptr(target_tokens), _ptr(n_accepted), _ptr(workspace), workspace.numel(), _stream(logits))
