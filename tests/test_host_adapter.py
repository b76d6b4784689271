"""The C++20 host adapter (oracle_amd/host) -- validation on CPU, full path on the GPU."""
import subprocess
from pathlib import Path

import pytest

EXE = Path(__file__).resolve().parents[1] / "oracle_amd" / "host" / "adapter_test"


def run(mode):
    if not EXE.exists():
        pytest.fail(f"{EXE} not built (run __graft_entry__.build())")
    proc = subprocess.run([str(EXE), mode], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert f"passed ({mode})" in proc.stdout


def test_adapter_validation_without_gpu():
    run("cpu")


@pytest.mark.gpu
def test_adapter_on_gpu():
    run("gpu")


REFERENCE_INCLUDE = "/root/reference/include"


@pytest.mark.skipif(not __import__("os").path.isdir(REFERENCE_INCLUDE), reason="reference headers not present")
def test_adapter_compiles_against_reference_types(tmp_path):
    """hip_quantized.hpp instantiated on the reference's GgufTensorView, StorageRowView and
    MappedGgufModel, from the reference's own headers (compile only)."""
    import subprocess
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    cmd = ["g++", "-std=c++20", "-fsyntax-only", "-Wall", "-Wextra", f"-I{REFERENCE_INCLUDE}",
           f"-I{root / 'include'}", f"-I{root / 'oracle_amd' / 'host'}", str(root / "tests" / "adapter_reference_compile.cpp")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
