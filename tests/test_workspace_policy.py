"""The context workspace growth policy (oracle_amd/csrc/oq_workspace.h), host only: an allocation
that a live captured graph may replay is retired instead of freed, growth during capture is
refused, and retired allocations are freed with the context's last graph; the capture refusal
(oq_capture_begin, or a caller's hipStreamBeginCapture on the context's stream) of
capture_in_progress.  Compiled with g++
against a counting allocator; no GPU."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_workspace_policy(tmp_path):
    exe = tmp_path / "workspace_policy_test"
    subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", f"-I{ROOT / 'oracle_amd' / 'csrc'}",
                    str(ROOT / "tests" / "workspace_policy_test.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
