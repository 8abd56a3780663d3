"""bench.py's command-line contract, on the CPU: one GPU only, refused before any GPU work."""
import os
import pathlib
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _bench(*args, env=None):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                          text=True, timeout=300, env={**os.environ, **(env or {})})


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr + r.stdout
    assert not r.stdout.strip().startswith("{"), "no result line may be printed"


def test_torchrun_world_size_is_refused():
    r = _bench("--gpus", "1", env={"WORLD_SIZE": "2", "RANK": "0", "LOCAL_RANK": "0"})
    assert r.returncode == 2
