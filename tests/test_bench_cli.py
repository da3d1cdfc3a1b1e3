"""bench.py's command line on the CPU: more than one GPU is refused with a
message and a non-zero exit before anything touches a device."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "1"],
                       stdout=subprocess.PIPE, stderr=subprocess.PIPE, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert b"one GPU only" in r.stderr
    assert r.stdout.strip() == b"", "no JSON line for a refused run"
