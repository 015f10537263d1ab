"""Runs the C++ forward test (tests/cpp/test_forward_hip.cc) on the GPU.

A small Qwen2-shaped model (2 layers, hidden 64, 4 query / 2 KV heads, int8
q/k/v/o/gate_up/down, tied fp32 embedding as LM head) runs a 20-token prompt
and 6 decode steps through the vvllm Backend and KVCache interfaces only, in
the operator order of the reference's transformer_forward
(include/vvllm/model/transformer.h:76-215), once on BackendHIP + KVCacheHIP
and once on a CPU Backend built from the oracle.  The logits are compared at
every step (fp32 activations: normalized error <= 1e-3; fp16: <= 5e-2 and the
same greedy token).
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_forward_hip_cpp():
    exe = os.path.join(ROOT, "tests", "cpp", "bin", "test_forward_hip")
    assert os.path.exists(exe), "tests/cpp/bin/test_forward_hip is not built (run __graft_entry__.build())"
    p = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(p.stdout)
    assert p.returncode == 0, p.stdout + p.stderr
