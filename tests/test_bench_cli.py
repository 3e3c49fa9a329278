"""CPU: bench.py measures one GPU.  Asked for more (--gpus N > 1, or launched as one rank of a
multi-rank job), it exits with status 2 and says why, before it touches a device."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def run(args, env=None):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([sys.executable, BENCH] + args, capture_output=True, text=True,
                          timeout=120, env=e, cwd=ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    r = run(["--gpus", "2"])
    assert r.returncode == 2
    assert "one GPU" in r.stderr and "--gpus 1" in r.stderr
    assert r.stdout == ""


def test_multi_rank_launch_exits_with_a_message():
    r = run([], env={"WORLD_SIZE": "4"})
    assert r.returncode == 2 and "one GPU" in r.stderr
