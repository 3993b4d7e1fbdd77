"""bench.py's command-line contract without a GPU: more than one GPU is
refused with a message, a machine without a GPU is refused too, and the
kernel-trace summary counts busy and idle time per step."""

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


def test_trace_summary_counts_busy_and_idle_time(tmp_path):
    """bench.py --summarize-trace: steps end at every second AdamW launch;
    overlapping kernels count once as busy time, the rest of the span is
    idle, and per-kernel time is averaged over the summarised steps."""
    import io
    import bench
    d = tmp_path / "trace" / "host"
    d.mkdir(parents=True)
    rows = ["Kernel_Name,Start_Timestamp,End_Timestamp"]
    t = 0
    for step in range(3):
        # two overlapping GEMMs (busy 0..150), a gap of 50, then the two AdamW launches
        rows += [f"void gemm_dl_kernel<1>(x),{t},{t + 100}",
                 f"gemm_dl_kernel<1>(x),{t + 50},{t + 150}",
                 f"adamw_kernel<float>(y),{t + 200},{t + 250}",
                 f"adamw_kernel<float>(y),{t + 250},{t + 300}"]
        t += 300
    (d / "kt_kernel_trace.csv").write_text("\n".join(rows) + "\n")
    out = io.StringIO()
    bench.summarize_trace(str(tmp_path / "trace"), 2, out=out)
    text = out.getvalue()
    # each summarised step spans 300 ns: busy 150 + 100, idle 50
    assert "mean per step: span 0.0 ms" in text
    lines = [l for l in text.splitlines() if l.startswith("| 0 |") or l.startswith("| 1 |")]
    assert len(lines) == 2
    assert "| `gemm_dl_kernel<1>` | 2 |" in text and "| `adamw_kernel<float>` | 2 |" in text


def test_counter_summary_derives_mfma_use_and_scaled_traffic(tmp_path):
    """bench.py --summarize-counters: per-kernel means over dispatches, MFMA
    utilisation from the busy cycles of 1024 SIMDs over GRBM_GUI_ACTIVE of 8
    XCDs, instructions per MFMA, and FETCH_SIZE / WRITE_SIZE scaled by what
    the 1 GiB calibration copy (the first copy dispatch; the fill that makes
    its source comes first) reads, each counter from its own pass."""
    import io
    import bench
    head = "Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value"
    sq = tmp_path / "a"
    sq.mkdir()
    rows = [head]
    for d in (1, 2):  # two dispatches of one kernel, per-XCD rows summed
        rows += [f"{d},void gemm_dl(x),SQ_VALU_MFMA_BUSY_CYCLES,512000",
                 f"{d},void gemm_dl(x),GRBM_GUI_ACTIVE,4000", f"{d},void gemm_dl(x),GRBM_GUI_ACTIVE,4000",
                 f"{d},void gemm_dl(x),SQ_INSTS_MFMA,100", f"{d},void gemm_dl(x),SQ_INSTS_VALU,150"]
    (sq / "p_counter_collection.csv").write_text("\n".join(rows) + "\n")
    passes = []
    for counter, fill, copy, gemm in (("FETCH_SIZE", 0, 524288, 1024),
                                      ("WRITE_SIZE", 1048576, 1048576, 2048)):
        tr = tmp_path / counter
        tr.mkdir()
        rows = [head, f"1,void fill(z),{counter},{fill}", f"2,__amd_rocclr_copyBuffer,{counter},{copy}",
                f"3,void gemm_dl(x),{counter},{gemm}"]
        (tr / "p_counter_collection.csv").write_text("\n".join(rows) + "\n")
        passes.append(str(tr))
    out = io.StringIO()
    bench.summarize_counters([str(sq), *passes], out=out)
    line = next(l for l in out.getvalue().splitlines() if l.startswith("| `gemm_dl`"))
    cells = [c.strip() for c in line.strip("|").split("|")]
    # 512000 busy cycles / (8000 / 8 * 1024) = 50 %; 150 VALU / 100 MFMA;
    # fetch 1024 KiB x 2 (the copy read 512 MiB of 1 GiB) = 2 MiB, write 2 MiB
    assert cells[1] == "2" and cells[2] == "50.0 %" and cells[3] == "1.50"
    assert cells[-2:] == ["2.0", "2.0"]
    # one GEMM launch of 2 + 2 MiB
    assert "traffic_bytes_per_launch: 4194304" in out.getvalue()
