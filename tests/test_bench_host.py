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


def test_gemm_bytes_covers_every_epilogue():
    """Every epilogue code the library exports has an algorithmic byte count:
    A and B read once in bf16, C written in its store type, plus the residual
    read or the float32 read-modify-write of an accumulated gradient."""
    sys.path.insert(0, str(ROOT))
    import bench
    from alodlm_amd import _lib
    M, N, K = 256, 512, 1024
    ab = 2 * (M * K + N * K)
    want = {_lib.EPI_STORE: ab + 2 * M * N, _lib.EPI_RESIDUAL: ab + 4 * M * N,
            _lib.EPI_ACCUM: ab + 8 * M * N, _lib.EPI_STORE_F32: ab + 4 * M * N}
    codes = {v for k, v in vars(_lib).items() if k.startswith("EPI_")}
    assert codes == set(want)
    for epi, nbytes in want.items():
        assert bench.gemm_bytes(None, 0, 0, None, 0, 0, None, 0, M, N, K, epi=epi) == nbytes
