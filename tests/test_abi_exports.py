"""CPU checks of the drop-in boundary: libtrc_hip.so loads and exports every
entry point include/trc_hip_abi.h declares, and the entry points that can run
without a GPU behave (no device -> clean errors, forced-error hook)."""
import re
import subprocess
import sys

import pytest

from conftest import ROOT
from traincpp_amd import hip as H

HEADER = ROOT / "include" / "trc_hip_abi.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(trc_hip_\w+)\s*\(", text, re.M)))


def test_header_declares_the_bound_entry_points():
    assert declared() == sorted(H.EXPORTS)


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", str(H.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    syms = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [s for s in declared() if s not in syms]
    assert not missing, missing
    lib = H.load()
    for s in declared():
        assert getattr(lib, s) is not None


def test_library_has_gfx950_code_objects():
    # the fat binary embedded by hipcc names its device code objects by target id
    assert b"amdgcn-amd-amdhsa--gfx950" in H.LIB_PATH.read_bytes()


def run_py(code: str, env=None):
    import os
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=e, cwd=str(ROOT / "tests"),
                          timeout=120)


def test_errors_without_a_device_are_clean():
    code = ("import conftest\nfrom traincpp_amd import hip as H\n"
            "n = H.device_count()\n"
            "if n == 0:\n"
            "    try:\n        H.init(0)\n    except H.HipError as e:\n        print('init', e.code)\n"
            "else:\n    print('init', 0)\n")
    r = run_py(code)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() in ("init -4", "init 0")


def test_forced_error_hook_on_cpu():
    code = ("import conftest\nfrom traincpp_amd import hip as H\n"
            "try:\n    H.device_count()\nexcept H.HipError as e:\n    print(e.code, H.last_error())\n")
    r = run_py(code, {"TRC_HIP_FORCE_ERROR": "trc_hip_device_count"})
    assert r.returncode == 0, r.stderr
    assert r.stdout.startswith("-5 trc_hip_device_count: forced failure")


@pytest.mark.parametrize("bad", [
    "H.check(H.load().trc_hip_dequant(12, None, 1, None, None))",
    "H.check(H.load().trc_hip_dequant(2, None, -1, None, None))",
    "H.check(H.load().trc_hip_qmatvec(2, None, 48, 1, 27, None, 1, 192, None, 4, None))",
    "H.check(H.load().trc_hip_malloc(None, 16))",
    # y overlapping W (rows of 36 bytes at 0x100000) or x (0x200000): refused
    # before any device work, so the fake addresses are never dereferenced
    "H.check(H.load().trc_hip_qmatvec(2, 0x100000, 64, 4, 36, 0x200000, 1, 256, 0x100040, 16, None))",
    "H.check(H.load().trc_hip_qmatvec(2, 0x100000, 64, 4, 36, 0x200000, 2, 256, 0x2000f0, 16, None))",
    # dst += mul_mat with one dst plane of 65536 x 32768 floats (8 GiB): over the
    # 2 GiB the accumulate kernels address, refused before any device work
    "H.mul_mat_acc_f32(H.tensor(0x100000, [4, 65536, 1, 1], H.contiguous_nb([4, 65536, 1, 1])), "
    "H.tensor(0x200000, [4, 32768, 1, 1], H.contiguous_nb([4, 32768, 1, 1])), "
    "H.tensor(0x1000000000, [65536, 32768, 1, 1], H.contiguous_nb([65536, 32768, 1, 1])))",
])
def test_argument_validation_precedes_device_work(bad):
    code = "import conftest\nfrom traincpp_amd import hip as H\ntry:\n    " + bad + \
           "\nexcept H.HipError as e:\n    print(e.code)\n"
    r = run_py(code)
    assert r.returncode == 0, r.stderr
    assert int(r.stdout.strip()) < 0
