"""Build the C++20 host adapter test program (oracle_amd/host/adapter_test).

The adapter itself (hip_quantized.hpp/.cpp) is source meant to be compiled into the host
application; the test program links it with liboq.so and, as the checker, the CPU oracle.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

HOST = Path(__file__).resolve().parent
PKG = HOST.parent
ROOT = PKG.parent
EXE = HOST / "adapter_test"


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "all"], check=True)
    tmp = EXE.with_name(EXE.name + ".tmp")
    cmd = [
        os.environ.get("CXX", "g++"), "-std=c++20", "-O2", "-Wall", "-Wextra",
        f"-I{ROOT / 'include'}",
        str(HOST / "hip_quantized.cpp"), str(HOST / "adapter_test.cpp"),
        f"-L{PKG}", "-loq", f"-L{ROOT / 'oracle'}", "-loracle",
        "-Wl,-rpath,$ORIGIN/..", "-Wl,-rpath,$ORIGIN/../../oracle",
        "-o", str(tmp),
    ]
    subprocess.run(cmd, check=True)
    os.replace(tmp, EXE)
    return EXE


if __name__ == "__main__":
    print(build())
