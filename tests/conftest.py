import importlib.util
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "train.cpp_amd"
GOLDEN = Path(__file__).resolve().parent / "golden"

sys.path.insert(0, str(Path(__file__).resolve().parent))


def load_pkg():
    """Imports train.cpp_amd/ (a directory name that is not an identifier) as traincpp_amd."""
    if "traincpp_amd" in sys.modules:
        return sys.modules["traincpp_amd"]
    spec = importlib.util.spec_from_file_location("traincpp_amd", PKG / "__init__.py",
                                                  submodule_search_locations=[str(PKG)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["traincpp_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


load_pkg()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


@pytest.fixture(scope="session")
def hip():
    """The C-ABI binding, initialised on device 0. Fails (never skips) when the
    library or the GPU is missing: GPU tests must exercise the native path."""
    from traincpp_amd import hip as h
    props = h.init(0)
    print(f"[hip] device 0: {props.name.decode()} {props.arch.decode()} CUs={props.compute_units}", flush=True)
    return h


@pytest.fixture
def tmp_dir(tmp_path):
    return str(tmp_path)


def announce(msg: str) -> None:
    """Names the case before a GPU step so a crash log says what was running."""
    print(f"[case] {msg}", flush=True)
    sys.stderr.flush()
