"""bench.py's command-line contract without a GPU: more than one GPU is
refused with a message, and a machine without a GPU is refused too."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=300)


def test_more_than_one_gpu_is_refused():
    out = run("--gpus", "2")
    assert out.returncode == 2
    assert "one GPU" in out.stderr


def test_cpu_only_machine_is_refused():
    import torch
    if torch.cuda.is_available():
        return
    out = run("--steps", "1", "--warmup", "0")
    assert out.returncode == 2
    assert "needs a GPU" in out.stderr


def test_model_choices():
    out = run("--model", "70b")
    assert out.returncode == 2 and "invalid choice" in out.stderr
