"""bench.py command-line contract on the CPU: more than one GPU is refused
with a message and exit status 2 before anything touches a GPU, and every
extra row can be named on its own."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_row_names_are_the_extra_rows():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--help"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0
    for row in ("cfg2_bs64_mixed", "cfg3_mtp3", "cfg4_indexshare", "lidu_init", "indexer_project",
                "prefill_persist"):
        assert row in r.stdout
