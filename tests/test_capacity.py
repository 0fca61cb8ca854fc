"""The launchers' host-side capacity checks, without a GPU.

Every launcher that writes a scratch buffer sized at ana_open (the split
attention's partials, the exact attention's scores, the GLA scan's regions,
the bf16 products' split activations) takes that buffer's capacity and
rejects a grid that needs more with hipErrorInvalidValue before launching,
and the decode paths that are switched off above four rows (the fast GLA
step and the flash-decoding attention) reject such steps the same way.
tests/capacity_probe.cpp calls the launchers of ana_amd/libana.so directly
with such arguments, on host placeholders: it runs with every device hidden
(HIP_VISIBLE_DEVICES and ROCR_VISIBLE_DEVICES), and refuses to run a case if
a device is still visible.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIBDIR = os.path.join(ROOT, "ana_amd")
CLANG = "/opt/rocm/llvm/bin/clang++"


@pytest.mark.skipif(not os.path.exists(CLANG), reason="amdclang++ not found")
def test_launchers_reject_oversized_grids(tmp_path):
    if not os.path.exists(os.path.join(LIBDIR, "libana.so")):
        pytest.skip("libana.so is not built")
    exe = str(tmp_path / "capacity_probe")
    subprocess.run([CLANG, "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    "-I" + os.path.join(LIBDIR, "csrc"), os.path.join(HERE, "capacity_probe.cpp"),
                    "-L" + LIBDIR, "-lana", "-L/opt/rocm/lib", "-lamdhip64",
                    "-Wl,-rpath," + LIBDIR, "-o", exe], check=True)
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", ROCR_VISIBLE_DEVICES="-1", CUDA_VISIBLE_DEVICES="-1")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120, env=env)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    if r.stdout.startswith("skip"):
        pytest.skip(r.stdout.strip())
    assert "0 failed" in r.stdout
