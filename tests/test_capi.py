"""CPU: the C-ABI library loads and exports every entry point include/dspark.h declares.
No kernel is launched (there may be no GPU); only the pure shape queries are called."""

from __future__ import annotations

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions() -> set[str]:
    text = open(os.path.join(ROOT, "include", "dspark.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(dspark_[a-z0-9_]+)\s*\(", text))


def test_header_and_binding_table_agree():
    from dspark_rocm import _lib

    assert _header_functions() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    from dspark_rocm import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libdspark_rocm.so is not built (run mlx-dspark_amd/build.py)")
    assert set(_lib.exported_symbols()) == _header_functions()
    lib = _lib.load()
    assert b"gfx950" in lib.dspark_version()


def test_shape_queries_without_gpu():
    from dspark_rocm import _lib

    lib = _lib.load()
    assert lib.dspark_qmm_affine_supported(16, 4096, 4096, 4, 64) == 0
    assert lib.dspark_qmm_affine_supported(16, 4096, 4096, 3, 64) == -6
    assert lib.dspark_qmm_affine_supported(16, 4000, 4096, 4, 64) == -2
    assert lib.dspark_verify_attention_workspace(1, 32, 8, 16, 128, 32784) > 0
    assert lib.dspark_verify_attention_blocks(1, 32, 8, 16, 128, 32784) > 1
    assert lib.dspark_verify_attention_blocks(1, 32, 8, 16, 100, 1024) == -1  # head_dim % 8 != 0
    assert lib.dspark_verify_attention_blocks(1, 32, 8, 16, 96, 1024) == \
        lib.dspark_verify_attention_blocks(1, 32, 8, 16, 128, 1024)            # the 128-column instance
    assert lib.dspark_moe_workspace(16, 2048, 768, 128, 8) > 0
    assert lib.dspark_moe_workspace(16, 2048, 768, 128, 64) == 0              # k > 32
    assert lib.dspark_last_error() is not None


def test_moe_packed_plan_picks_the_per_cu_kernel_for_verify_widths():
    """The packed MoE block runs its gate/up projection one workgroup per CU for M <= 16 tokens,
    E <= 256, M * k <= 512 and the instantiated widths (K = H in {512, 2048}); every other shape,
    and the down projection always, keeps one workgroup per (expert, strip)."""
    from dspark_rocm import ops

    cu, rc = ops.MOE_KERNELS[1], ops.MOE_KERNELS[0]
    for bits in (4, 8):
        assert ops.moe_packed_plan(16, 2048, 768, 128, 8, bits) == {"gate_up": cu, "down": rc}
        assert ops.moe_packed_plan(1, 2048, 768, 256, 8, bits) == {"gate_up": cu, "down": rc}
        assert ops.moe_packed_plan(16, 512, 256, 2, 2, bits) == {"gate_up": cu, "down": rc}
        assert ops.moe_packed_plan(16, 2048, 1536, 128, 8, bits) == {"gate_up": cu, "down": rc}
        assert ops.moe_packed_plan(17, 2048, 768, 128, 8, bits)["gate_up"] == rc   # M > 16
        assert ops.moe_packed_plan(16, 2048, 768, 257, 8, bits)["gate_up"] == rc   # E > 256
        assert ops.moe_packed_plan(16, 2048, 768, 128, 33, bits)["gate_up"] == rc  # M * k > 512
        assert ops.moe_packed_plan(16, 256, 128, 8, 2, bits)["gate_up"] == rc
        assert ops.moe_packed_plan(16, 4096, 768, 128, 8, bits)["gate_up"] == rc


def test_plan_blocks_scale_with_length():
    from dspark_rocm import _lib

    lib = _lib.load()
    nb = [lib.dspark_verify_attention_blocks(1, 32, 8, 16, 128, L + 16) for L in (512, 4096, 16384, 32768)]
    assert nb == sorted(nb) and nb[0] >= 1
    # every block covers whole 64-key tiles and the blocks cover the cache
    assert lib.dspark_verify_attention_workspace(1, 32, 8, 16, 128, 64) == 0   # one block: no partials


def test_split_k_plans_never_leave_a_slice_empty():
    """Every plan the library picks cuts K into S non-empty slices that fit the kernel
    instantiation (an empty slice would make the kernel read the group before its first one).
    The cut (multiples of 8 groups when G % 8 == 0, else of 2 for 4-bit rows, else 1, slice
    sl starting at unit * floor(sl * units / S)) is checked as a partition of [0, G)."""
    import ctypes

    from dspark_rocm import _lib

    lib = _lib.load()
    out = (ctypes.c_int32 * 4)()
    checked = 0
    for bits in (4, 8):
        for g in list(range(1, 80)) + [96, 128, 160, 192, 256, 320, 384, 400, 512]:
            K = 64 * g
            for N in (16, 64, 1024, 4096, 6144, 151936):
                for M in (1, 16, 64):
                    if lib.dspark_qmm_affine_plan(M, K, N, bits, 64, out) != 0:
                        continue
                    S, ksmax = out[0], out[1]
                    unit = 8 if g % 8 == 0 else 2 if bits == 4 else 1
                    units = -(-g // unit)
                    cuts = [min(unit * ((sl * units) // S), g) for sl in range(S + 1)]
                    sizes = [b - a for a, b in zip(cuts, cuts[1:])]
                    assert cuts[0] == 0 and cuts[-1] == g, (bits, K, N, M, S)
                    assert min(sizes) >= 1 and max(sizes) <= ksmax, (bits, K, N, M, S, sizes)
                    checked += 1
    assert checked > 1000


def test_noalloc_qmm_refuses_oversize_before_any_gpu_call():
    """A shape whose split-K scratch exceeds the library-held array is refused on the host
    (DSPARK_ERR_WORKSPACE) before any HIP call: the pointers below are never dereferenced."""
    from dspark_rocm import _lib

    lib = _lib.load()
    N, K, M = 151936, 5120, 16
    assert lib.dspark_qmm_affine_workspace(M, K, N, 8, 64) > (256 << 10) + (32 << 20)
    fake = 1 << 20  # 256-byte aligned, non-null; never touched
    st = lib.dspark_qmm_affine_noalloc(fake, K, M, K, fake, fake, fake, N, 8, 64, fake, N, None)
    assert st == -4
    assert b"scratch" in lib.dspark_last_error()
    # a shape that fits passes the same host checks (it would then need a GPU to launch)
    assert lib.dspark_qmm_affine_workspace(16, 25600, 5120, 8, 64) <= (256 << 10) + (32 << 20)
    assert lib.dspark_qmm_affine_workspace(16, 5120, 2 * 25600, 8, 64) <= (256 << 10) + (32 << 20)
