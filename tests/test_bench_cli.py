"""bench.py's command line on the CPU: one GPU only.  Every GPU box here has
one GPU, so ``--gpus N`` with N above 1 must exit with a message that says so
(and a non-zero status) before touching a device."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert proc.returncode != 0
    assert "one GPU only" in proc.stdout + proc.stderr
