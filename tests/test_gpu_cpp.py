"""The C++ interface (lite_ssm::MetalOps / DeviceBuffer / UnifiedBuffer, built
from include/lite_ssm/*.hpp) on the GPU: tests/cpp/test_metal_ops.cpp checks
every reference kernel name and runs rmsnorm / int4 GEMV from a mmap'd file /
a batch / ssd_step against the CPU oracle."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_cpp_metal_ops():
    exe = os.path.join(ROOT, "tests", "cpp", "_bin", "test_metal_ops")
    assert os.path.exists(exe), "tests/cpp/_bin/test_metal_ops not built"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
