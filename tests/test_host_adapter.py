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
