"""Build recipe for the in-tree native libraries (no cmake/ninja needed).

    libtrc_hip.so       HIP kernels for gfx950 + the extern "C" ABI of
                        include/trc_hip_abi.h (hipcc, one object per .hip file)
    libtraincpp_hip.so  the traincpp-compatible C++ core subset plus the HIP
                        Device/BufferType/Buffer implementation, linked against
                        libtrc_hip.so (g++)

Outputs go to train.cpp_amd/lib/. Every call rebuilds from source.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
LIB = PKG / "lib"
OBJ = PKG / "lib" / "obj"
HIP_SRC = PKG / "csrc" / "hip"
CORE_SRC = PKG / "csrc" / "core"
BACKEND_SRC = PKG / "csrc" / "backend"
INCLUDE = ROOT / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("TRC_HIP_ARCH", "gfx950")

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}", f"-I{HIP_SRC}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
# Per-file extras. Dequantization must round every * and + on its own.
HIP_FILE_FLAGS = {"dequant.hip": ["-ffp-contract=off"]}

CXX = os.environ.get("CXX", "g++")
# -ffp-contract=off: the host dequantizer (core/gguf.cpp) rounds d*q and +m on their own.
CXX_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-ffp-contract=off", f"-I{INCLUDE}", f"-I{CORE_SRC}", "-Wall", "-Wextra",
             "-Wno-unused-parameter"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"build step failed: {' '.join(cmd[:3])} ... ({res.returncode})")
    elif verbose and res.stderr.strip():
        # hipcc's host pass warns that it does not know the packed-fp32 feature.
        lines = [l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l]
        if lines:
            sys.stderr.write("\n".join(lines) + "\n")


def build_hip(verbose: bool = False, jobs: int = 8) -> Path:
    OBJ.mkdir(parents=True, exist_ok=True)
    srcs = sorted(HIP_SRC.glob("*.hip"))
    objs = []
    cmds = []
    for s in srcs:
        o = OBJ / (s.stem + ".o")
        objs.append(o)
        cmds.append([HIPCC, *HIP_FLAGS, *HIP_FILE_FLAGS.get(s.name, []), "-c", str(s), "-o", str(o)])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    out = LIB / "libtrc_hip.so"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(out)], verbose)
    return out


def build_core(verbose: bool = False, jobs: int = 8) -> Path | None:
    srcs = sorted(CORE_SRC.glob("*.cpp")) + sorted(BACKEND_SRC.glob("*.cpp"))
    if not srcs:
        return None
    OBJ.mkdir(parents=True, exist_ok=True)
    objs = []
    cmds = []
    for s in srcs:
        o = OBJ / ("core_" + s.stem + ".o")
        objs.append(o)
        cmds.append([CXX, *CXX_FLAGS, "-c", str(s), "-o", str(o)])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    out = LIB / "libtraincpp_hip.so"
    _run([CXX, "-shared", "-fPIC", *map(str, objs), f"-L{LIB}", "-ltrc_hip", "-Wl,-rpath,$ORIGIN",
          "-o", str(out)], verbose)
    return out


def build_all(verbose: bool = False) -> None:
    LIB.mkdir(parents=True, exist_ok=True)
    build_hip(verbose)
    build_core(verbose)


if __name__ == "__main__":
    build_all(verbose="-v" in sys.argv)
