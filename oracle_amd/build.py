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


# Sources compiled more than once, with different macro definitions: one object per entry.
# oq_gemv_inst.hip holds the K-quant GEMV instantiations of one (weight type, activation form).
VARIANTS = {
    "oq_gemv_inst.hip": [
        (f"t{t}_{'f32' if fused else 'q8k'}", [f"-DOQ_KQ_TYPE={t}", f"-DOQ_KQ_FUSED={int(fused)}"])
        for t in (12, 13, 14) for fused in (True, False)
    ],
}


def units() -> list[tuple[Path, Path, list[str]]]:
    """(source, object, extra flags) for every object of liboq.so."""
    out = []
    for src in sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp")):
        for tag, flags in VARIANTS.get(src.name, [("", [])]):
            name = src.name + (f".{tag}" if tag else "") + ".o"
            out.append((src, OBJ / name, flags))
    return out


def _stale(obj: Path, src: Path) -> bool:
    if not obj.exists():
        return True
    deps = [src, *CSRC.glob("*.h"), ROOT / "include" / "oq.h", Path(__file__)]
    return any(d.stat().st_mtime > obj.stat().st_mtime for d in deps)


CALIBRATION = PKG / "calibration"


def _build_calibration(force: bool) -> None:
    """The HBM read-floor program (calibration/read_floor.hip), a standalone executable."""
    src = CALIBRATION / "read_floor.hip"
    exe = CALIBRATION / "read_floor"
    if not force and exe.exists() and exe.stat().st_mtime >= src.stat().st_mtime:
        return
    _run([HIPCC, *DEVICE_FLAGS, "-x", "hip", str(src), "-o", str(exe)])


def build(jobs: int = 8, force: bool = True) -> Path:
    """Compile every translation unit (force=False: only objects older than their sources or
    any header) and link liboq.so."""
    OBJ.mkdir(exist_ok=True)
    todo = [u for u in units() if force or _stale(u[1], u[0])]
    objs = [u[1] for u in units()]

    def compile_one(unit):
        src, obj, flags = unit
        lang = ["-x", "hip"] if src.suffix == ".hip" else []
        _run([HIPCC, *DEVICE_FLAGS, *flags, *lang, "-c", str(src), "-o", str(obj)])

    # the longest units first
    todo.sort(key=lambda u: (u[0].name != "oq_gemv_inst.hip", u[0].name != "oq_gemv_block.hip"))
    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(todo) or 1))) as pool:
        list(pool.map(compile_one, todo))
    _build_calibration(force)
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(force="--incremental" not in sys.argv))
