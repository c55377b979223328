"""bench.py's command line on the CPU: it measures one GPU only, so --gpus N > 1 (or a multi-rank launch) exits at
once with a message and a non-zero status, before touching a GPU."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(*args, env=None):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True, timeout=120,
                          cwd=ROOT, env=env)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2")
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


def test_a_multi_rank_launch_is_refused():
    env = dict(os.environ, WORLD_SIZE="2", RANK="0", LOCAL_RANK="0")
    r = _run(env=env)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
