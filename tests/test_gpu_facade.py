"""The C++ operator facade (include/qw_ops.hpp) on the GPU: runs the
tests/cpp/test_facade program (built by __graft_entry__.build()), which
drives HipMLP / HipLMHead / HipGreedyArgmaxSampler / HipRMSNorm and the
attention projection classes exactly as the reference's caller drives its
CudaMLP / CudaLMHead / ... and checks each against the CPU oracle."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_facade")


@pytest.mark.gpu
def test_cpp_facade():
    assert os.path.exists(BIN), "tests/cpp/test_facade is not built: run __graft_entry__.build()"
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FACADE OK" in r.stdout
