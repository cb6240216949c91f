"""bench.py's contract on the CPU side: more than one GPU is refused with a
message (the path runs on one MI355X), before any GPU work."""
import subprocess
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr and proc.stdout == ""
