"""Builds the C++ drop-in test program tests/cpp/bin/test_hip_backend against
libtraincpp_hip.so (the backend under test) and oracle/liboracle.so (the checker)."""
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent


def main() -> None:
    out = HERE / "bin" / "test_hip_backend"
    out.parent.mkdir(exist_ok=True)
    cmd = ["g++", "-std=c++20", "-O2", "-Wall", "-Wextra", "-Wno-unused-parameter",
           f"-I{ROOT / 'include'}", f"-I{ROOT / 'oracle'}", str(HERE / "test_hip_backend.cpp"),
           f"-L{ROOT / 'train.cpp_amd' / 'lib'}", "-ltraincpp_hip", "-ltrc_hip",
           f"-L{ROOT / 'oracle'}", "-l:liboracle.so",
           "-Wl,-rpath,$ORIGIN/../../../train.cpp_amd/lib", "-Wl,-rpath,$ORIGIN/../../../oracle",
           "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise SystemExit(r.returncode)


if __name__ == "__main__":
    main()
