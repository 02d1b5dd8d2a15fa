"""bench.py's command-line contract, on the CPU (no GPU work is started)."""
import subprocess
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent


def run_bench(*args):
    return subprocess.run([sys.executable, str(REPO / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    result = run_bench("--gpus", "2")
    assert result.returncode == 2
    assert "one GPU" in result.stderr and result.stdout == ""


def test_existing_output_file_is_never_overwritten(tmp_path):
    report = tmp_path / "report.json"
    report.write_text("keep me")
    result = run_bench("--output", str(report))
    assert result.returncode == 2
    assert "never overwrites" in result.stderr
    assert report.read_text() == "keep me"


def test_invalid_step_counts_are_refused():
    assert run_bench("--steps", "0").returncode == 2
    assert run_bench("--warmup", "-1").returncode == 2
