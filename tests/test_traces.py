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


def test_position_hash_content_detects_misplaced_bytes():
    """The synthetic expert content the bench verifies slots against: every word differs
    within a slab and across experts, layers and buffers; chunked generation equals one-shot
    generation; and a slot holding another expert's row, another layer's, or one 16-byte
    vector shifted is reported as a mismatch."""
    import torch

    from vllm_expert_cache import traces

    nbytes, E = 256, 6
    rows = {(l, b): traces.expert_words(l, range(E), b, nbytes, "cpu")
            for l in (0, 1) for b in (0, 1)}
    allw = torch.cat([r.flatten() for r in rows.values()])
    assert allw.unique().numel() == allw.numel()
    part = traces.expert_words(1, [4], 1, nbytes, "cpu", first_word=8, nwords=20)
    assert torch.equal(part[0], rows[(1, 1)][4, 8:28])
    store = torch.empty(E * nbytes, dtype=torch.uint8)
    traces.fill_expert_store(store, 1, 0, nbytes, E, "cpu", chunk_words=7)
    assert torch.equal(store.view(torch.int32).view(E, -1), rows[(1, 0)])

    se = torch.tensor([2, -1, 5, 0], dtype=torch.int32)
    slots = torch.zeros(4, nbytes // 4, dtype=torch.int32)
    for s, e in enumerate(se.tolist()):
        if e >= 0:
            slots[s] = rows[(1, 0)][e]
    flat = slots.view(torch.uint8).flatten()
    for cw in (3, 64, 1 << 20):
        assert traces.slots_match(flat, se, 1, 0, nbytes, chunk_words=cw) == (True, 3)
    bad = [slots.clone() for _ in range(3)]
    bad[0][2] = rows[(1, 0)][4]                     # another expert's row
    bad[1][0] = rows[(0, 0)][2]                     # the same expert of another layer
    bad[2][3, 8:12] = rows[(1, 0)][0, 12:16]        # one 16-byte vector shifted
    for b in bad:
        assert traces.slots_match(b.view(torch.uint8).flatten(), se, 1, 0, nbytes,
                                  chunk_words=3)[0] is False
