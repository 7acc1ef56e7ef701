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


def test_committed_profiles_feed_the_bench_line():
    """The counter summaries the JSON line quotes (roofline.traffic, manage_remap_counters)
    load, and their figures hang together: traffic is fetch plus write per one-expert
    launch, within a few percent of the algorithmic bytes."""
    sys.path.insert(0, str(ROOT))
    import bench

    t, m = bench._traffic(), bench._manage_counters()
    assert t is not None and m is not None
    assert t["bytes_per_launch"] == t["fetch_bytes_per_miss"] + t["write_bytes_per_miss"]
    assert t["write_bytes_per_miss"] == t["algorithmic_bytes_per_miss"] == 4732928
    assert 1.0 <= t["fetch_over_algorithmic"] < 1.05
    assert m["hbm_bytes_read"] > 0 and m["hbm_bytes_written"] > 0 and m["kernel_us"] > 0
    # GB/s over the stamped kernel time
    assert abs(m["hbm_GBps"] - (m["hbm_bytes_read"] + m["hbm_bytes_written"]) /
               (m["kernel_us"] * 1e3)) < 0.05


def test_committed_bench_lines_are_verified_runs():
    """Every bench JSON line kept under profiles/ is a run of this bench that verified itself
    (slot bytes and the oracle's per-step miss lists and final state) and reports a gather
    fraction no larger than the link peak it measured."""
    import json

    sys.path.insert(0, str(ROOT))
    import bench

    files = sorted((ROOT / "profiles").glob("bench-*.json"))
    assert files
    for f in files:
        rec = json.loads(f.read_text())
        line = rec["line"]
        assert rec["command"].startswith("python3 bench.py"), f.name
        assert line["metric"] == bench.METRIC
        assert line["verified"]["all"] is True, f.name
        for k in ("slot_bytes", "state", "n_miss_per_step", "miss_lists_per_step"):
            assert line["verified"][k] is True, (f.name, k)
        assert 0.5 < line["roofline"]["frac"] <= 1.0, f.name
        assert f.name == f"bench-{line['config']['workload']}.json" or \
            f.name.startswith(f"bench-{line['config']['workload']}-"), f.name


def test_stamps_library_exports():
    """bench_stamps.so, when built, exports the stamped kernels' entry points the bench
    binds."""
    import ctypes

    import pytest

    path = ROOT / "bench_stamps.so"
    if not path.is_file():
        pytest.skip("bench_stamps.so not built (run __graft_entry__.build())")
    h = ctypes.CDLL(str(path))
    for name in ("stamped_manage_remap", "stamped_gather", "stamped_empty",
                 "stamped_clock_khz"):
        assert hasattr(h, name), name


def test_substitution_windows_count_only_their_chunks():
    """The decode chain's figures per window: chunks end at every cut, so the timed window
    (steps 5..25 inside a pass 5..4096 timed in chunks of 16) sums exactly its own steps,
    and the per-node costs come out of synthetic chunk times whose per-step costs are
    known: a policy node adding 2.4 us, an empty node 1.5 us, the gathers moving each
    step's inserts at a fixed rate plus 1.5 us per node."""
    sys.path.insert(0, str(ROOT))
    import bench

    pts = bench.chunk_points(5, 4096, 16, cuts=(2048, 25))
    assert pts[0] == 5 and pts[-1] == 4096 and 25 in pts and 2048 in pts
    assert pts[:4] == [5, 16, 25, 32]
    assert bench.chunk_points(5, 25, 16, cuts=(25, 4000)) == [5, 16, 25]

    L, B, rate = 48, 4732928, 55e9
    nm = np.zeros((4096, L), np.int64)
    nm[5:25] = 2
    nm[25:] = np.arange(4096 - 25)[:, None] % 2
    g = nm.sum(1) * B / rate + L * 1.5e-6           # gathers-only graph, per step
    per_step = {"gathers": g, "gathers_again": g, "empty+gather": g + L * 1.5e-6,
                "full": g + L * 2.4e-6, "policy": np.full(4096, L * 2.5e-6)}
    times = {k: [(c0, c1, float(v[c0:c1].sum())) for c0, c1 in zip(pts[:-1], pts[1:])]
             for k, v in per_step.items()}
    for lo, hi in ((5, 25), (5, 4096), (2048, 4096)):
        w = bench.substitution_window(times, lo, hi, nm, L, B, 57.6)
        assert w["trace_steps"] == [lo, hi]
        assert w["inserts"] == int(nm[lo:hi].sum())
        assert w["manage_remap_us_per_layer"] == 2.4
        assert w["empty_node_us"] == 1.5
        assert w["manage_remap_over_empty_node_us"] == 0.9
        assert w["noise_us_per_layer"] == 0.0
        assert w["policy_graph_us_per_layer"] == 2.5
        gather_s = float((g[lo:hi] - L * 0.1e-6).sum())
        assert w["gather_GBps"] == round(float(nm[lo:hi].sum()) * B / gather_s / 1e9, 3)
        assert abs(w["gather_us_per_launch"] - gather_s * 1e6 / ((hi - lo) * L)) < 1e-3
