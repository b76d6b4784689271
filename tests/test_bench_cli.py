"""bench.py's command line on the CPU: a request for more than one GPU exits with status 2 and a
message before any device work (this build times one GPU only)."""

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def run_bench(*args, env=None):
    e = dict(os.environ, **(env or {}))
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, env=e, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = run_bench("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout.strip() == ""


def test_extra_ranks_exit_quietly():
    r = run_bench("--steps", "1", "--warmup", "0", env={"WORLD_SIZE": "4"})
    assert r.returncode == 2 and r.stdout.strip() == ""
