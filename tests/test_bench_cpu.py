"""bench.py's contract pieces that need no GPU: one GPU only, and the counter
probe's shape strings."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], cwd=REPO, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""  # no JSON line


def test_pmc_shape_strings():
    sys.path.insert(0, str(REPO))
    import bench

    assert bench.parse_pmc_shape("1x5120x17408") == (1, 5120, 17408)
    assert bench.parse_pmc_shape("32x17408x5120") == (32, 17408, 5120)
    assert bench.parse_pmc_shape("r2g128x17408x5120") == ("rowwise", 2, 128, 17408, 5120)
    assert bench.parse_pmc_shape("r8g64x4096x4096") == ("rowwise", 8, 64, 4096, 4096)
