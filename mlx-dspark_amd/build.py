"""Build the gfx950 HIP library (``dspark_rocm/libdspark_rocm.so``) from ``csrc/*.hip``.

One shared object with C linkage (``include/dspark.h``); every translation unit is compiled by
``hipcc --offload-arch=gfx950`` in parallel, then linked. Always recompiles (the build check
must exercise the compiler), writing to a temporary file that replaces the library atomically.

    python mlx-dspark_amd/build.py [--jobs N] [--verbose]
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OUT = os.path.join(HERE, "dspark_rocm", "libdspark_rocm.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    # no packed fp32 arithmetic in device code (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: accumulator registers would cost a v_accvgpr move per
    # value on every rescale / scale-FMA (and an occupancy step for the 4-wave attention)
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]

# Extra flags of single translation units
FILE_FLAGS = {
    # the per-CU MoE expert kernel unrolls its unit loops in full (up to 68 steps of one 1 KB
    # load each), past LLVM's default full-unroll threshold; a loop left partly rolled would
    # index the kernel's load window at run time and keep it in scratch memory
    "dspark_moe_cu.hip": ["-mllvm", "-pragma-unroll-threshold=200000"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the dspark kernels)")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str, obj: str, verbose: bool) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(jobs: int | None = None, verbose: bool = False) -> str:
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no .hip sources under {CSRC}")
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with tempfile.TemporaryDirectory(prefix="dspark_build_") as tmp:
        objs = [os.path.join(tmp, os.path.basename(s) + ".o") for s in srcs]
        with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
            futs = [ex.submit(_compile, s, o, verbose) for s, o in zip(srcs, objs)]
            for f in futs:
                f.result()
        tmp_out = OUT + ".tmp"
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_out]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stderr}")
        os.replace(tmp_out, OUT)
    return OUT


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))


if __name__ == "__main__":
    main()
