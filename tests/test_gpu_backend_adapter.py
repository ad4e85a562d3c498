"""HipBackend through the reference's ExecutionBackend interface (GPU).

Runs tests/cpp/hip_backend_test, built by __graft_entry__.build() against the
reference's headers (neural-network_amd/backend/Makefile): the Tensor-style
op calls of src/core/tensor.cpp on HipBackend, checked against the
reference's known answers (tensor_test.cpp, layer_test.cpp), the oracle's
Dense product and LayerNorm (bit for bit) and closed forms; then the C++
decoder objects HipDecoder / HipKVCache against the oracle (forward logits,
the KV cache and truncate, greedy speculative decoding in fp32, INT8 and
INT4).
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROGRAM = os.path.join(ROOT, "tests", "cpp", "hip_backend_test")

pytestmark = pytest.mark.gpu


@pytest.mark.skipif(not os.path.exists(PROGRAM),
                    reason="built only where the reference's headers are "
                           "present (__graft_entry__.build)")
def test_hip_backend_program():
    r = subprocess.run([PROGRAM], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "checks passed" in r.stdout
