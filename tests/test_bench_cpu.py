"""bench.py's contract on the host: it measures one GPU and says so when
asked for more (the build has no multi-GPU path), before touching a GPU."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def _run(*args, env=None):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, env=env, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2 and r.stdout == ""
    assert "one GPU" in r.stderr


def test_a_multi_rank_launch_is_refused():
    env = dict(os.environ, WORLD_SIZE="4", RANK="0", LOCAL_RANK="0")
    r = _run("--gpus", "1", env=env)
    assert r.returncode == 2 and "one GPU" in r.stderr
