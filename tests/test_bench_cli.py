"""The bench's command line: it measures one GPU, so a request for more (the flag, or a launcher's WORLD_SIZE)
exits with status 2 and a message, before touching torch or a GPU."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_bench(args, env_extra=None):
    env = dict(os.environ, **(env_extra or {}))
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=60, env=env)  # fmt: skip


def test_more_than_one_gpu_refused():
    r = run_bench(["--gpus", "2"])
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_launcher_world_size_refused():
    r = run_bench(["--gpus", "1"], {"WORLD_SIZE": "8"})
    assert r.returncode == 2
    assert "one GPU" in r.stderr
