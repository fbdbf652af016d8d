"""CPU checks of the C++ side of the boundary: the traincpp-compatible core in
libtraincpp_hip.so (layouts, views, graph order, GGUF parsing and corrupt-file
rejection) through tests/cpp/bin/test_hip_backend --cpu, the mul_mat shape
guard as a death test (the reference's tests/test_mul_mat_shape_guard.cpp), and
that the HIP Device source compiles against the reference's own public
headers, i.e. drops into the reference tree unchanged."""
import shutil
import os
import subprocess
from pathlib import Path

import pytest

from conftest import ROOT

BIN = ROOT / "tests" / "cpp" / "bin" / "test_hip_backend"
REFERENCE_INCLUDE = Path("/root/reference/include")


def test_core_without_device(tmp_path):
    r = subprocess.run([str(BIN), "--cpu"], capture_output=True, text=True, timeout=120,
                       env={**os.environ, "TMPDIR": str(tmp_path)})
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS" in r.stdout


def test_mul_mat_shape_guard_aborts():
    r = subprocess.run([str(BIN), "--abort-shape"], capture_output=True, text=True, timeout=60)
    assert r.returncode != 0
    assert "inner dimensions differ" in r.stderr


@pytest.mark.skipif(not (REFERENCE_INCLUDE / "traincpp" / "trc_backend.h").exists(),
                    reason="reference checkout not present")
def test_hip_device_compiles_against_reference_headers(tmp_path):
    # the plugin's own two headers beside the reference's (what a maintainer copies)
    abi = tmp_path / "abi"
    (abi / "traincpp").mkdir(parents=True)
    shutil.copy(ROOT / "include" / "trc_hip_abi.h", abi)
    shutil.copy(ROOT / "include" / "traincpp" / "trc_hip.h", abi / "traincpp")
    r = subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-Wall", "-Wextra", "-Wno-unused-parameter",
                        f"-I{REFERENCE_INCLUDE}", f"-I{abi}",
                        str(ROOT / "train.cpp_amd" / "csrc" / "backend" / "hip_device.cpp")],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
