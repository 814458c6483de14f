"""GPU: dspark_qmm_affine_noalloc (no workspace argument, library-held split-K scratch) against
dspark_qmm_affine with a caller workspace, through the C ABI: bit-identical outputs on two calls
in a row, the second with a smaller input, and after dspark_qmm_noalloc_reset has cleared
counters left stale. (The refusal of a shape too large for the scratch is
a host-side check, tested on the CPU in test_capi.py.)"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import qmm_ref, quant_ref
from _util import from_dev_bf16, rng, to_dev_bf16, to_dev_packed


def _problem(r, M, N, K, bits, dev):
    x = quant_ref.bf16_round(r.standard_normal((M, K)).astype(np.float32))
    w, s, b = quant_ref.random_packed(r, N, K, bits)
    return x, (w, s, b), (to_dev_bf16(x, dev), to_dev_packed(w, dev), to_dev_bf16(s, dev), to_dev_bf16(b, dev))


def _with_workspace(lib, xd, wd, sd, bd, M, N, K, bits, stream):
    from dspark_rocm import _lib

    y = torch.empty((M, N), dtype=torch.bfloat16, device=xd.device)
    nbytes = int(lib.dspark_qmm_affine_workspace(M, K, N, bits, 64))
    ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=xd.device)
    _lib.call("dspark_qmm_affine", xd.data_ptr(), K, M, K, wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), N, bits, 64,
              y.data_ptr(), N, ws.data_ptr(), ws.numel(), stream)
    return y


def _noalloc(xd, wd, sd, bd, M, N, K, bits, stream):
    from dspark_rocm import _lib

    y = torch.empty((M, N), dtype=torch.bfloat16, device=xd.device)
    _lib.call("dspark_qmm_affine_noalloc", xd.data_ptr(), K, M, K, wd.data_ptr(), sd.data_ptr(), bd.data_ptr(), N,
              bits, 64, y.data_ptr(), N, stream)
    return y


def _workspace_bytes(lib, M, N, K, bits):
    return int(lib.dspark_qmm_affine_workspace(M, K, N, bits, 64))


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_twice(dev):
    from dspark_rocm import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    r = rng(71)
    # first call: a split-K shape with many slices; second: smaller input (fewer rows, a
    # narrower and shallower matrix, other bits), so stale partials of the first call sit past
    # the second call's region of the shared scratch. Both plans use the scratch (a non-zero
    # workspace), so a plan change that drops split-K cannot empty the test.
    for M, N, K, bits in ((16, 6144, 4096, 8), (5, 1024, 2048, 4)):
        assert _workspace_bytes(lib, M, N, K, bits) > 0, (M, N, K, bits)
        print(f"noalloc M={M} N={N} K={K} bits={bits}", flush=True)
        x, (w, s, b), (xd, wd, sd, bd) = _problem(r, M, N, K, bits, dev)
        want = _with_workspace(lib, xd, wd, sd, bd, M, N, K, bits, stream)
        got = _noalloc(xd, wd, sd, bd, M, N, K, bits, stream)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"M={M} N={N} K={K} bits={bits}"
        ref = qmm_ref.qmm(x, w, s, b, bits)
        err = float(np.max(np.abs(from_dev_bf16(got) - ref)))
        assert err <= 2e-2 * float(np.sqrt(np.mean(np.asarray(ref, np.float64) ** 2)))


class _Raw:
    """A device byte range as a torch tensor (no allocation: the library's own array)."""

    def __init__(self, ptr: int, n: int):
        self.__cuda_array_interface__ = {"shape": (n,), "typestr": "|u1", "data": (ptr, False), "version": 3}


@pytest.mark.gpu
def test_noalloc_reset_clears_stale_counters(dev):
    """Counters left stale (as a call that did not complete would leave them: here written
    from the host side) are cleared by dspark_qmm_noalloc_reset; the next call is bitwise the
    workspace entry point's, and leaves the counters at zero."""
    import ctypes

    from dspark_rocm import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    ptr, nbytes = ctypes.c_void_p(), ctypes.c_size_t()
    _lib.call("dspark_qmm_noalloc_scratch", ctypes.byref(ptr), ctypes.byref(nbytes))
    torch.cuda.synchronize()
    assert ptr.value and nbytes.value >= (256 << 10) + (32 << 20)
    counters = torch.as_tensor(_Raw(ptr.value, 256 << 10), device=dev)
    assert counters.data_ptr() == ptr.value
    counters.fill_(7)
    torch.cuda.synchronize()
    _lib.call("dspark_qmm_noalloc_reset", stream)
    torch.cuda.synchronize()
    assert not counters.any()
    M, N, K, bits = 16, 6144, 4096, 4   # a split-K plan ([4096, 4096] runs whole-K, no scratch)
    assert _workspace_bytes(lib, M, N, K, bits) > 0
    x, (w, s, b), (xd, wd, sd, bd) = _problem(rng(72), M, N, K, bits, dev)
    want = _with_workspace(lib, xd, wd, sd, bd, M, N, K, bits, stream)
    got = _noalloc(xd, wd, sd, bd, M, N, K, bits, stream)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert not counters.any()
