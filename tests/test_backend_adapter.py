"""The C++ drop-in layer compiles against the reference's own headers (CPU).

neural-network_amd/backend holds HipBackend (an ExecutionBackend,
include/backend/backend.hpp:20-221) and the decoder objects (HipDecoder,
HipKVCache, HipQuantizedDense; include/nn/layer.hpp:212-330,
include/nn/quantization.hpp:15-43) over libnnhip.so's C ABI.  Compiling them
with the reference's headers checks every override against the reference's
signatures (HipBackend is `final` and instantiated by the test program, so a
missing or mistyped virtual is a compile error).  Skipped where the
reference tree is absent (its headers are not part of this repository).
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INCLUDE = "/root/reference/include"
BACKEND = os.path.join(ROOT, "neural-network_amd", "backend")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_INCLUDE),
                                reason="the reference's headers are absent")


def compile_only(src, tmp_path, extra=()):
    out = tmp_path / (os.path.basename(src) + ".o")
    cmd = ["g++", "-std=c++20", "-Wall", "-Wextra", "-Werror", "-c",
           f"-I{REF_INCLUDE}", f"-I{os.path.join(ROOT, 'include')}",
           f"-I{BACKEND}", *extra, src, "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    return out


@pytest.mark.parametrize("name", ["hip_backend.cpp", "hip_nn.cpp"])
def test_adapter_compiles_against_reference_headers(name, tmp_path):
    compile_only(os.path.join(BACKEND, name), tmp_path)


def test_backend_test_program_compiles(tmp_path):
    """The GPU test program instantiates HipBackend through ExecutionBackend&
    (every pure virtual overridden)."""
    compile_only(os.path.join(ROOT, "tests", "cpp", "hip_backend_test.cpp"),
                 tmp_path, extra=(f"-I{os.path.join(ROOT, 'neural-network_amd')}",))
