"""bench.py on the CPU: it measures one GPU and refuses --gpus N > 1 with a
message (this path has no cross-GPU work), its shape helpers are the reference's, and its
prefetch predictors and segment windows are what the measurements describe."""
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


def test_prefetch_predictions_and_segment_spread():
    """The prefetch leg's predictors: accuracy 1.0 is the true routing; at 0.8 about a fifth
    of the ids are replaced, by any expert ("uniform") or by one the same layer routes
    elsewhere in the trace ("routed"). Segment starts stay inside their window."""
    sys.path.insert(0, str(ROOT))
    import bench
    from vllm_expert_cache import traces

    w = traces.WORKLOADS["48-layer-e128"]
    ids = np.stack([traces.routing(w, l, 600) for l in range(4)], axis=1)  # [T, L, mk]
    assert np.array_equal(bench._predictions(np, ids, 100, 400, w.experts, 1.0, "uniform"),
                          ids[100:500])
    for errors in ("uniform", "routed"):
        pred = bench._predictions(np, ids, 100, 400, w.experts, 0.8, errors)
        assert pred.shape == (400, 4, w.mk)
        assert pred.min() >= 0 and pred.max() < w.experts
        same = (pred == ids[100:500]).mean()
        assert 0.78 < same < 0.86, (errors, same)
        if errors == "routed":
            for l in range(4):
                assert set(np.unique(pred[:, l])) <= set(np.unique(ids[:, l]))
    for lo, hi, n, length in ((5, 25, 8, 2), (2048, 4096, 8, 8), (0, 10, 3, 20), (7, 9, 1, 1)):
        starts = bench._spread(lo, hi, n, length)
        assert starts == sorted(set(starts)) and len(starts) <= max(1, n)
        assert all(lo <= s and (s + length <= hi or s == lo) for s in starts)
