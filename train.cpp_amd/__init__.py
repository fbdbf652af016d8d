"""traincpp MI355X HIP backend: Python-side helpers.

The product is native: libtrc_hip.so (HIP kernels + C ABI, include/trc_hip_abi.h)
and libtraincpp_hip.so (the traincpp Device/BufferType/Buffer plugin in C++).
This package holds the build recipe (build.py), the ctypes binding of the C ABI
(hip.py) and the seeded synthetic input generator (synth.py).
"""
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_DIR = PKG_DIR / "lib"
