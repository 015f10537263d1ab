"""Runs the C++ BackendHIP test (tests/cpp/test_backend_hip.cc) on the GPU.

It drives the MI355X backend through the vvllm Backend interface, restating
the reference's own linear_q8 tests (src/backend/backend_naive_test.cc:
355-425) in fp32 and fp16 mode, plus the in-place linear_q8_add the model
uses and the weight-mirror refresh.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_backend_hip_cpp():
    exe = os.path.join(ROOT, "tests", "cpp", "bin", "test_backend_hip")
    assert os.path.exists(exe), "tests/cpp/bin/test_backend_hip is not built (run __graft_entry__.build())"
    p = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(p.stdout)
    assert p.returncode == 0, p.stdout + p.stderr
