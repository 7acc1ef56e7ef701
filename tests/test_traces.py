"""Routing-trace generators (csrc/traces.c) and the replay format.

Properties the workloads promise: deterministic per (workload, layer); ids in range and
distinct within a token; Zipf skew and the stated repeat probability; the group limit of
the grouped workload; round trip through the reference's npz replay format.
"""
from __future__ import annotations

import numpy as np
import pytest

from vllm_expert_cache import traces

W = traces.WORKLOADS


def test_deterministic_and_layer_seeded():
    w = W["48-layer-e128"]
    a, b = traces.routing(w, 5, 300), traces.routing(w, 5, 300)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, traces.routing(w, 6, 300))
    # layer 0 of the 48-layer workload is the single-layer workload
    assert np.array_equal(traces.routing(W["single-layer-e128"], 0, 300),
                          traces.routing(w, 0, 300))


@pytest.mark.parametrize("name", sorted(W))
def test_shape_range_and_distinct_per_token(name):
    w = W[name]
    ids = traces.routing(w, 0, 200)
    assert ids.shape == (200, w.mk) and ids.dtype == np.int32
    assert ids.min() >= 0 and ids.max() < w.experts
    per_tok = ids.reshape(200, w.tokens, w.top_k)
    for row in per_tok.reshape(-1, w.top_k):
        assert len(set(row.tolist())) == w.top_k


def test_repeat_probability_and_skew():
    w = W["single-layer-e128"]
    ids = traces.routing(w, 0, 4096)
    kept = [len(set(ids[t]) & set(ids[t - 1])) for t in range(1, len(ids))]
    # each previous expert is kept with p=0.6; a fresh Zipf draw can also re-pick one
    assert 0.6 * 8 <= np.mean(kept) <= 0.6 * 8 + 1.0
    counts = np.bincount(ids.ravel(), minlength=128)
    top = np.sort(counts)[::-1]
    assert top[:8].sum() > 0.25 * counts.sum()      # skewed
    assert (counts > 0).sum() > 100                   # but broad


def test_uniform_routing_of_the_large_expert_workload():
    w = W["8-layer-e8-bf16"]
    ids = traces.routing(w, 0, 4000)
    counts = np.bincount(ids.ravel(), minlength=8) / ids.size
    assert np.abs(counts - 1 / 8).max() < 0.02


def test_group_limit():
    w = W["8-layer-e256-fp8"]
    ids = traces.routing(w, 0, 50).reshape(50, w.tokens, w.top_k)
    gs = w.experts // w.groups
    for tok in ids.reshape(-1, w.top_k):
        assert len(set((tok // gs).tolist())) <= w.topk_groups


def test_expert_byte_layouts():
    assert W["48-layer-e128"].bytes_per_expert == 4_732_928
    assert W["8-layer-e8-bf16"].bytes_per_expert == 352_321_536
    assert W["8-layer-e256-fp8"].bytes_per_expert == 44_050_944
    for w in W.values():
        assert all(b.nbytes % 16 == 0 for b in w.buffers)


def test_routes_npz_round_trip(tmp_path):
    ids = np.stack([traces.routing(W["48-layer-e128"], l, 20) for l in range(3)], axis=1)
    ids[3, 1, 2:] = -1
    p = tmp_path / "routes.npz"
    traces.save_routes(str(p), ids)
    back = traces.load_routes(str(p))
    assert back.shape == (20, 3, 8) and np.array_equal(back, ids)


def test_bench_counts_distinct_experts_without_padding():
    """bench.py's hit rate divides by the distinct routed experts of each (step, layer); on a
    recorded trace the -1 padding is not an expert."""
    import sys
    from pathlib import Path

    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    import bench

    ids = np.array([[[3, 3, -1, 5], [-1, -1, -1, -1]], [[1, 2, 3, 4], [0, 0, 0, 0]]], np.int32)
    assert bench._distinct(np, ids).tolist() == [[2, 0], [4, 1]]
    rng = np.random.default_rng(0)
    big = rng.integers(-1, 40, size=(50, 3, 12)).astype(np.int32)
    want = [[len(set(r[r >= 0].tolist())) for r in step] for step in big]
    assert bench._distinct(np, big).tolist() == want
