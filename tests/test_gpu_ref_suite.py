"""The reference's own golden and gradient-golden programs (tests/test_golden.cpp,
tests/test_grad_golden.cpp of the reference, compiled unchanged into
oracle/_ref/test_ref_suite by oracle/Makefile `suite`) run against the HIP device:
every golden case whose graph the device supports must match the PyTorch golden
data at the tolerances those programs set (tests/test_golden.cpp:190-201); the
others are reported as skipped by the programs' own graph_first_unsupported
check. The golden data are the reference's fixtures in tests/golden/reference_suite."""
import subprocess

import pytest

from conftest import ROOT, announce

BIN = ROOT / "oracle" / "_ref" / "test_ref_suite"

pytestmark = pytest.mark.gpu


@pytest.mark.skipif(not BIN.exists(), reason="oracle/_ref not built (reference checkout absent at build time)")
def test_reference_golden_programs_on_the_hip_device(hip):
    announce("reference golden + grad-golden programs on the HIP device")
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=600, cwd=str(ROOT))
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert "2 cases run, 0 failed" in r.stdout
    ran = [l for l in r.stdout.splitlines() if "[ OK ]" in l]
    assert len(ran) >= 4, "expected the supported golden cases (add, mul, mul_mat, ...) to run"
    ok = {l.split("[ OK ]", 1)[1].split()[0] for l in ran if l.split("[ OK ]", 1)[1].split()}
    # the mul_mat gradient goldens (sum(sqr(mul_mat)) and its backward through
    # scale, mul, repeat_back, acc and the transposed products) and the unary
    # goldens of the two ops that path needs
    for case in ("mul_mat", "mul_mat_batch", "mul_mat_batch_bcast_div", "grad_mul_mat_batch",
                 "grad_mul_mat_batch_div", "unary_sqr", "scale"):
        assert case in ok, f"golden case {case} did not run on the HIP device"
