"""bench.py's command line on the CPU: it measures one GPU only and refuses
more, and it rejects unknown workloads and invalid step counts, before
touching a device."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_exits_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_world_size_above_one_exits_too():
    env = dict(os.environ, WORLD_SIZE="2")
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")], capture_output=True, text=True, timeout=120,
                       env=env)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_invalid_step_counts_are_refused():
    for args in (("--steps", "0"), ("--warmup", "-1"), ("--settle-ms", "-5")):
        r = _run(*args)
        assert r.returncode == 2 and "--steps must be at least 1" in r.stderr, args
