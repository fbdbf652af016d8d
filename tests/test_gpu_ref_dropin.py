"""The HIP backend dropped into the REFERENCE library: tests/cpp/test_ref_dropin.cpp,
linked with the reference's own core, autograd, liveness allocator, GGUF reader
and CPU device (compiled from the reference's sources into oracle/_ref by
oracle/Makefile's `ref` and `dropin` targets). It runs a Linear layer with bias
forward + backward built by the reference's graph_build_backward_expand,
allocated by buffer_alloc_graph_tensors and cleared by graph_reset, at the
4096 x 4096 x 512 benchmark shape, and the GGUF Q8_0 4096 x 4096 warm start
through the reference's gguf_load_tensor and through hip_gguf_load_tensor.
Bars (written in the program): y, dW, dX within 1e-4 row-L2 of the oracle; db,
the loss and the dequantized weights bit for bit; small graphs within the
reference's conformance tolerance of its own CPU device."""
import os
import subprocess

import pytest

from conftest import ROOT, announce

BIN = ROOT / "oracle" / "_ref" / "test_ref_dropin"

needs_bin = pytest.mark.skipif(not BIN.exists(), reason="oracle/_ref not built (reference checkout absent at build time)")


@needs_bin
def test_selfcheck_on_the_reference_cpu_device(tmp_path):
    """The program's oracle compositions against the reference's CPU device
    standing in for the GPU (no GPU needed)."""
    r = subprocess.run([str(BIN), "--cpu-selfcheck"], capture_output=True, text=True, timeout=300, cwd=tmp_path)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert "ALL PASSED" in r.stdout


@pytest.mark.gpu
@needs_bin
def test_linear_autograd_and_gguf_on_the_reference_core(hip, tmp_path):
    announce("reference core + HIP device: Linear fwd+bwd 4096x4096x512, GGUF Q8_0 warm start")
    r = subprocess.run([str(BIN), str(tmp_path / "cfg0.gguf")], capture_output=True, text=True, timeout=600,
                       cwd=tmp_path)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert "ALL PASSED" in r.stdout
    fused = [l for l in r.stdout.splitlines() if "result digest" in l]
    assert len(fused) == 1

    # The same program with the plugin's fusion of dW's chain (mul_mat -> transpose
    # -> cont -> acc into W's accumulator, run as one product added into it) turned
    # off: every check passes node by node too, and y, dW, dX and db are the same bits.
    announce("the same, dW's chain node by node (TRC_HIP_NO_FUSION=1)")
    r2 = subprocess.run([str(BIN), str(tmp_path / "cfg0b.gguf")], capture_output=True, text=True, timeout=600,
                        cwd=tmp_path, env={**os.environ, "TRC_HIP_NO_FUSION": "1"})
    print(r2.stdout)
    assert r2.returncode == 0, r2.stdout[-4000:] + r2.stderr[-2000:]
    assert "ALL PASSED" in r2.stdout
    assert [l for l in r2.stdout.splitlines() if "result digest" in l] == fused
