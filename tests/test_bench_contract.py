"""bench.py's command-line contract on the CPU: one GPU only, refused before
anything touches a device."""
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _run(args, env_extra=None):
    env = dict(os.environ, **(env_extra or {}))
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT, env=env,
                          capture_output=True, text=True, timeout=300)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run(["--gpus", "2"])
    assert r.returncode == 2 and "one GPU only" in r.stderr


def test_a_multi_rank_launch_is_refused_with_a_message():
    r = _run(["--gpus", "1"], {"WORLD_SIZE": "8"})
    assert r.returncode == 2 and "one GPU only" in r.stderr
