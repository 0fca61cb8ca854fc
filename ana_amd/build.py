"""Build libana.so (gfx950) in-tree with hipcc.

Flags that matter for the numerics: -ffp-contract=off keeps every product
and the sum it joins two roundings (the reference's CPU kernels compile the
same way, bend/effs/bulk.c:30-35), and -packed-fp32-ops keeps the compiler
from emitting packed FP32 instructions.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libana.so")
SOURCES = ["ana.hip", "kernels_exact.hip", "kernels_fast.hip", "gemm_wide.hip", "sampler.hip", "decode_persist.hip",
           "ftc2.cpp", "bpe.cpp"]
OBJDIR = os.path.join(HERE, "_build")


def hipcc() -> str:
    for p in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if p and os.path.exists(p):
            return p
    raise RuntimeError("hipcc not found")


def flags() -> list[str]:
    return [
        "--offload-arch=gfx950", "-O3", "-fPIC", "-shared", "-std=c++17",
        "-ffp-contract=off", "-fno-fast-math",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function", "-Wno-unused-result",
    ]


def build(verbose: bool = False) -> str:
    """Compile every source (in parallel) and link ana_amd/libana.so; always
    recompiles."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(OBJDIR, exist_ok=True)
    compile_flags = [f for f in flags() if f != "-shared"]

    def one(src: str) -> str:
        obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
        cmd = [hipcc(), *compile_flags, "-c", "-o", obj, os.path.join(CSRC, src)]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n" + r.stdout + r.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(one, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), *flags(), "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
