"""bench.py's command-line contract on the CPU: more than one GPU is refused
with a message (this build measures one GPU), and the documented flags parse."""

import subprocess
import sys

from .conftest import ROOT


def _run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr + r.stdout


def test_documented_flags_parse():
    r = _run("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--no-block", "--no-rollout", "--no-halo", "--no-backward", "--no-cpu"):
        assert flag in r.stdout, flag
