"""bench.py's command-line contract that needs no GPU: it measures one GPU
only, so any other --gpus (or a WORLD_SIZE above 1) exits with status 2 and a
message before touching a device."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]


def _run(args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, str(REPO / "bench.py"), *args], capture_output=True,
                          text=True, timeout=120, env=env)


def test_more_than_one_gpu_is_refused():
    out = _run(["--gpus", "2", "--steps", "5", "--warmup", "1"])
    assert out.returncode == 2, out
    assert "one GPU only" in out.stderr
    assert out.stdout == ""


def test_world_size_above_one_is_refused():
    out = _run(["--steps", "5"], {"WORLD_SIZE": "8"})
    assert out.returncode == 2
    assert "WORLD_SIZE 8" in out.stderr


def test_help_lists_the_contract_flags():
    out = _run(["--help"])
    assert out.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup"):
        assert flag in out.stdout
