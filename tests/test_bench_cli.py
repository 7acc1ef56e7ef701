"""bench.py's command line on the CPU: it measures one GPU and refuses --gpus N > 1 with a
message (this path has no cross-GPU work), and its shape helpers are the reference's."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused_with_a_message():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 2
    assert "measures one GPU" in res.stderr
    assert res.stdout == ""  # no JSON line for a run that did not happen


def test_align_lengths_match_the_oracle_tests():
    sys.path.insert(0, str(ROOT))
    import bench
    from test_oracle import align_lengths

    for mk, E, bs in ((8, 128, 16), (32, 128, 16), (128, 256, 16), (300, 128, 4), (1, 8, 1)):
        assert bench._align_lengths(mk, E, bs) == align_lengths(mk, E, bs)
    assert np.array_equal(bench._distinct(np, np.array([[[-1, -1]]])), [[0]])
