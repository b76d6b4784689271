"""Build recipe for liboq.so (the gfx950 kernels + C ABI) and the C++ host adapter test.

Compiles every translation unit under oracle_amd/csrc with hipcc for gfx950 only, in-tree, and
links oracle_amd/liboq.so.  Packed-FP32 instruction selection is disabled for device code.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "liboq.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed: {cmd[-1]}")
    noise = "is not a recognized feature for this target"
    for line in (proc.stdout + proc.stderr).splitlines():
        if line.strip() and noise not in line:
            sys.stderr.write(line + "\n")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def build(jobs: int = 8) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = sources()
    objs = [OBJ / (s.name + ".o") for s in srcs]

    def compile_one(pair):
        src, obj = pair
        lang = ["-x", "hip"] if src.suffix == ".hip" else []
        _run([HIPCC, *DEVICE_FLAGS, *lang, "-c", str(src), "-o", str(obj)])

    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as pool:
        list(pool.map(compile_one, zip(srcs, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())
