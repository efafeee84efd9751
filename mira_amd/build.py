"""Build libmira_rocm.so (the gfx950 kernels and their C ABI) in-tree with hipcc.

    python -m mira_amd.build          # compiles mira_amd/libmira_rocm.so

Flags that matter for bit-exact parity with MIRA's NumPy golden model:
  -ffp-contract=off                         no a*b+c -> fma contraction in epilogues
  -fhip-fp32-correctly-rounded-divide-sqrt  IEEE f32 division in the quantizer
  (no -ffast-math, denormals kept)
and for this hardware: packed-fp32 instructions disabled (-packed-fp32-ops).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libmira_rocm.so"
ARCH = "gfx950"

SOURCES = ["abi.hip", "quantize.hip", "qgemm.hip", "qgemv.hip", "w8gemm.hip", "misc.hip", "stem.hip", "decode.hip", "expand_dw.hip", "loop.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-rdc",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the fused epilogue unrolls over every MFMA block a wave holds; without a
    # higher threshold the unroller gives up and the accumulators go to scratch
    "-mllvm", "-pragma-unroll-threshold=100000",
    "-Wall",
    "-Wno-unused-result",
    f"-I{ROOT / 'include'}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the rocm target needs ROCm's hipcc to build libmira_rocm.so")


def build(verbose: bool = False, jobs: int = 4) -> Path:
    """Compile every source to an object in parallel, then link the shared library."""
    cc = hipcc()
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    procs = []
    objs = []
    for src in SOURCES:
        obj = objdir / (Path(src).stem + ".o")
        objs.append(obj)
        cmd = [cc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        if len([p for _, p in procs if p.poll() is None]) >= jobs:
            procs[0][1].wait()
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        if p.returncode != 0:
            failed.append(f"--- {src}\n{out}")
        elif verbose and out.strip():
            print(out)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n".join(failed))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(f"built {path}")
