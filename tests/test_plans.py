"""CPU check of the engine's and the persistent kernel's launch plans
(tests/c/plan_main.cpp): every decode-shape GEMM launch the batched engine can
plan uses an instantiated kernel and fits the split-K buffers sized for the
model, and the role split is valid for every grid size.  Built with hipcc for
the host only; no GPU is touched."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_launch_plans(tmp_path):
    exe = tmp_path / "plan_main"
    src = os.path.join(ROOT, "tests", "c", "plan_main.cpp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O1", "-std=c++17", "-I" + os.path.join(ROOT, "dnn.c_amd", "csrc"),
           "-I" + os.path.join(ROOT, "include"), src, "-o", str(exe)]
    b = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert b.returncode == 0, b.stderr[-3000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "plans ok" in r.stdout, r.stdout[-3000:]
