"""Builds the C++ test drivers under tests/cpp/_build/ (test infrastructure, run by the tests).

hip_engine_test links libember_hip.so (the product library, built first) and drives ember::create_backend("hip")
with the engine's page logic; it is built here on the CPU and run by a GPU test. g++ compiles it from the product
headers: the C++ classes cross the library boundary with the Itanium ABI and the shared libstdc++ both sides use.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
BUILD = HERE / "_build"
LIB_DIR = ROOT / "ember_amd"


def hip_engine_test() -> Path:
    gxx = shutil.which("g++")
    if gxx is None:
        raise RuntimeError("g++ is required to build the C++ test drivers")
    BUILD.mkdir(exist_ok=True)
    out = BUILD / "hip_engine_test"
    cmd = [gxx, "-std=c++20", "-O1", "-Wall", "-Wextra", f"-I{ROOT / 'ember_amd' / 'csrc' / 'host'}",
           f"-I{ROOT / 'include'}", f"-I{HERE}", str(HERE / "hip_engine_test.cpp"), f"-L{LIB_DIR}", "-lember_hip",
           "-Wl,-rpath,$ORIGIN/../../../ember_amd", "-Wl,-rpath-link,/opt/rocm/lib", "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building {out.name} failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return out


def build() -> None:
    hip_engine_test()


if __name__ == "__main__":
    build()
