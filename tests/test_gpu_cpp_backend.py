"""The HIP Device through the traincpp API on the GPU: conformance mul_mat
graphs, linear-layer backward compositions (with bias, broadcast weight planes
and gradient accumulators: add / repeat_back / acc), GGUF warm start (configuration 0)
and quantized tensors in graphs, each against the CPU oracle
(tests/cpp/test_hip_backend.cpp)."""
import os
import subprocess

import pytest

from conftest import ROOT, announce

pytestmark = pytest.mark.gpu

BIN = ROOT / "tests" / "cpp" / "bin" / "test_hip_backend"


def test_backend_through_traincpp_api(tmp_path):
    announce("C++ drop-in backend test")
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=600,
                       env={**os.environ, "TMPDIR": str(tmp_path)})
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert "PASS: 0 failure(s)" in r.stdout
    assert "add/repeat_back/acc bit-exact: yes" in r.stdout
