"""Prefetch on the GPU: expert_cache_prefetch against the oracle, and ExpertSlotCache's
prefetch -> refresh sequence through the side stream.

Kernel parity: each step runs prefetch(prediction) then manage(routing), the plugin's
order, on one layer's state; after every call the miss list, n_miss and the full state
(table, map_cold, slot_expert, slot_stamp, step) must equal the oracle's, bit for bit. The
cases reach every launch variant (slots per lane 1-16, table chunks 1-8, experts beyond
the LDS table), both victim searches (few inserts: wave-min; many: threshold select, with
32- and 64-bit stamp spreads), insert budgets of 0, 1 and S, and predictions that are right,
partly wrong or all wrong (ids outside [0, E) included).

End to end: the prefetched copy runs on a side stream while the current stream proceeds;
after the next refresh every resident slot must hold its expert's bytes, eagerly and in
HIP-graph replays checked against an eager twin.
"""
from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle
from test_gpu_cache import NAMES, Owner
from vllm_expert_cache.cache import ExpertSlotCache

pytestmark = pytest.mark.gpu

LRU, LFU = 0, 1

# name, E, S, mk, prefetch budget, policy, decay, prediction accuracy, initial stamps
CASES = [
    ("e128-s64", 128, 64, 8, 64, LFU, 64, 0.7, None),
    ("e128-s64-lru-right", 128, 64, 8, 64, LRU, 64, 1.0, None),
    ("e8-s4", 8, 4, 2, 4, LFU, 64, 0.5, None),
    ("e256-s128", 256, 128, 128, 128, LFU, 64, 0.7, None),
    ("e512-s257", 512, 257, 50, 64, LRU, 0, 0.6, None),
    ("e1000-s1024", 1000, 1024, 200, 1024, LFU, 3, 0.5, None),
    ("e5000-s300", 5000, 300, 64, 300, LRU, 0, 0.6, None),
    ("e128-s16-budget1", 128, 16, 8, 1, LFU, 64, 0.7, None),
    ("e128-s16-budget0", 128, 16, 8, 0, LRU, 64, 0.7, None),
    ("e257-s65-wide", 257, 65, 64, 65, LFU, 64, 0.0, "wide"),
    ("e64-s129-neg", 64, 129, 33, 129, LFU, 0, 0.5, "neg"),
]


def _routing(E, mk, T, rng):
    """Locality routing: each previous id kept with p 0.6, the rest Zipf draws; a few
    padding ids (-1)."""
    w = np.arange(1, E + 1, dtype=float) ** -1.1
    w /= w.sum()
    perm = rng.permutation(E)
    ids = np.zeros((T, mk), np.int32)
    prev = perm[rng.choice(E, mk, p=w)]
    for t in range(T):
        keep = rng.random(mk) < 0.6
        row = np.where(keep, prev, perm[rng.choice(E, mk, p=w)])
        row[rng.random(mk) < 0.03] = -1
        ids[t] = row
        prev = row
    return ids


def _predict(ids, E, acc, rng):
    """Each routed id kept with probability acc, else replaced by an id in [-2, E + 2)."""
    pred = ids.copy()
    wrong = rng.random(ids.shape) >= acc
    pred[wrong] = rng.integers(-2, E + 2, int(wrong.sum()))
    return pred


def _initial_stamps(kind, S, rng):
    if kind == "wide":
        return rng.integers(0, 1 << 45, S)
    if kind == "neg":
        return rng.integers(-(1 << 40), 1 << 40, S)
    return None


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_prefetch_then_manage_matches_oracle(case):
    name, E, S, mk, budget, policy, decay, acc, stamps = case
    T = 200
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    ids = _routing(E, mk, T, rng)
    pred = _predict(ids, E, acc, rng)
    init = _initial_stamps(stamps, S, rng)
    cap = max(S, budget, 1)
    print(f"case {name}: E={E} S={S} mk={mk} budget={budget} acc={acc}", flush=True)

    # GPU: one layer's state; the prefetch has its own miss list
    h = gu.lib()
    st = gu.Layers(1, E, S, miss_cap=cap)
    if init is not None:
        st.slot_stamp[0].copy_(torch.as_tensor(init, device=gu.DEV))
    pf_miss = torch.zeros((2 * cap,), dtype=torch.int32, device=gu.DEV)
    pf_n = torch.zeros((1,), dtype=torch.int32, device=gu.DEV)
    d_ids = torch.as_tensor(ids, device=gu.DEV)
    d_pred = torch.as_tensor(pred, device=gu.DEV)
    words = oracle.state_words(E, S)
    rec = {k: torch.zeros(shape, dtype=torch.int32, device=gu.DEV) for k, shape in (
        ("pf_n", (T,)), ("pf_miss", (T, 2 * cap)), ("pf_state", (T, words)),
        ("n", (T,)), ("miss", (T, 2 * cap)), ("state", (T, words)))}
    md = min(E, mk)
    for t in range(T):
        rc = h.expert_cache_prefetch(
            gu.P(d_pred[t].data_ptr()), mk, E, S, budget, st.row("table", 0),
            st.row("map_cold", 0), st.row("slot_expert", 0), st.row("slot_stamp", 0),
            st.row("routed", 0), gu.ptr(pf_miss), gu.ptr(pf_n), gu.stream())
        assert rc == 0, rc
        rec["pf_n"][t] = pf_n[0]
        rec["pf_miss"][t].copy_(pf_miss)
        rec["pf_state"][t].copy_(st.state_words()[0])
        rc = gu.manage_call(h, st, 0, gu.P(d_ids[t].data_ptr()), mk, md, S, policy, decay)
        assert rc == 0, rc
        rec["n"][t] = st.n_miss[0, 0]
        rec["miss"][t].copy_(st.miss[0])
        rec["state"][t].copy_(st.state_words()[0])
    torch.cuda.synchronize()
    got = {k: v.cpu().numpy() for k, v in rec.items()}

    # oracle: the same sequence, with the two miss lists kept apart
    ref = oracle.State(E, S, miss_cap=cap)
    if init is not None:
        ref.slot_stamp[:] = init
    pf_buf, pf_nb = np.zeros(2 * cap, np.int32), np.zeros(1, np.int32)
    want = {k: np.zeros_like(v) for k, v in got.items()}
    for t in range(T):
        real_miss, real_n = ref.miss.copy(), ref.n_miss.copy()
        ref.miss[:], ref.n_miss[:] = pf_buf, pf_nb
        assert ref.prefetch(pred[t], budget) == 0
        pf_buf, pf_nb = ref.miss.copy(), ref.n_miss.copy()
        ref.miss[:], ref.n_miss[:] = real_miss, real_n
        want["pf_n"][t] = pf_nb[0]
        want["pf_miss"][t] = pf_buf
        want["pf_state"][t] = _words(ref)
        assert ref.manage(ids[t], md, S, policy, decay) == 0
        want["n"][t] = ref.n_miss[0]
        want["miss"][t] = ref.miss
        want["state"][t] = _words(ref)

    for k in ("pf_n", "pf_miss", "pf_state", "n", "miss", "state"):
        d = gu.first_diff(got[k], want[k])
        assert d is None, f"{name}: {k} differs first at {d}: {got[k][d]} != {want[k][d]}"
    fetched = int(want["pf_n"].sum())
    print(f"  prefetched {fetched} experts, real inserts {int(want['n'].sum())}", flush=True)
    if budget > 0 and acc > 0:
        assert fetched > 0


def _words(s: oracle.State) -> np.ndarray:
    return np.concatenate([s.table, s.map_cold, s.slot_expert, s.slot_stamp.view(np.int32),
                           s.step.view(np.int32)])


def test_prefetch_rejects_bad_arguments():
    h = gu.lib()
    st = gu.Layers(1, 8, 4)
    for E, S, mi, mk in ((0, 4, 4, 1), (8, 0, 4, 1), (8, 1025, 4, 1), (8, 4, -1, 1),
                         (8, 4, 1025, 1), (8, 4, 4, -1)):
        rc = h.expert_cache_prefetch(gu.P(1), mk, E, S, mi, st.row("table", 0),
                                     st.row("map_cold", 0), st.row("slot_expert", 0),
                                     st.row("slot_stamp", 0), st.row("routed", 0),
                                     st.row("miss", 0), st.row("n_miss", 0), gu.stream())
        assert rc == -1, (E, S, mi, mk)


E, S, K = 128, 32, 8


def _all_slots_hold_their_experts(cache: ExpertSlotCache, src: dict):
    se = cache.slot_expert
    live = torch.nonzero(se >= 0).flatten()
    experts = se[live].long()
    for n in NAMES:
        assert torch.equal(cache.slots[n][live], src[n][experts]), n


def _device_sources(owner):
    return {n: getattr(owner, n).to(gu.DEV) for n in NAMES}


@pytest.mark.parametrize("policy", ["lfu", "lru"])
def test_cache_prefetch_then_refresh(monkeypatch, policy):
    monkeypatch.setenv("EXPERT_CACHE_POLICY", policy)
    owner = Owner(2)
    src = _device_sources(owner)
    cache = ExpertSlotCache(owner, NAMES, E, S, gu.DEV)
    ref = oracle.State(E, S)
    pol = 1 if policy == "lfu" else 0
    rng = np.random.default_rng(12)
    busy = torch.randn((2048, 2048), device=gu.DEV)
    for t in range(60):
        tokens = 1 + t % 4
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(tokens)]).astype(np.int32)
        pred = _predict(ids, E, 0.7 if t % 3 else 0.0, rng).astype(np.int64)
        assert cache.prefetch(torch.as_tensor(pred, device=gu.DEV))
        busy = busy @ busy.T * 1e-3  # current-stream work the copy overlaps
        slot_ids = cache.refresh(torch.as_tensor(ids, device=gu.DEV))
        assert ref.prefetch(pred.astype(np.int32), S) == 0
        assert ref.manage(ids.ravel(), min(E, ids.size), S, pol, 64) == 0
        torch.cuda.synchronize()
        assert np.array_equal(slot_ids.cpu().numpy().ravel(),
                              oracle.remap(ids.ravel(), ref.table)), t
        for f in ("table", "map_cold", "slot_expert", "slot_stamp", "step"):
            assert np.array_equal(getattr(cache, f).cpu().numpy(), getattr(ref, f)), (t, f)
        _all_slots_hold_their_experts(cache, src)
    assert not cache.prefetch(torch.zeros((5, K), dtype=torch.int32, device=gu.DEV))


def test_cache_prefetch_under_graph_capture():
    owner = Owner(3)
    src = _device_sources(owner)
    eager = ExpertSlotCache(owner, NAMES, E, S, gu.DEV)
    graphed = ExpertSlotCache(owner, NAMES, E, S, gu.DEV)
    for c in (eager, graphed):
        for buf in c.slots.values():
            buf.zero_()
    rng = np.random.default_rng(21)
    static_ids = torch.zeros((2, K), dtype=torch.int32, device=gu.DEV)
    static_pred = torch.zeros((2, K), dtype=torch.int32, device=gu.DEV)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for c in (graphed, eager):
            c.prefetch(static_pred)
            c.refresh(static_ids)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        graphed.prefetch(static_pred)
        static_out = graphed.refresh(static_ids)

    for t in range(40):
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(2)]).astype(np.int32)
        pred = _predict(ids, E, 0.6, rng)
        static_ids.copy_(torch.as_tensor(ids, device=gu.DEV))
        static_pred.copy_(torch.as_tensor(pred, device=gu.DEV))
        g.replay()
        eager.prefetch(static_pred.clone())
        want = eager.refresh(static_ids.clone())
        torch.cuda.synchronize()
        assert torch.equal(static_out, want), t
        for f in ("table", "map_cold", "slot_expert", "slot_stamp", "step", "pf_miss",
                  "pf_n_miss", "miss", "n_miss"):
            assert torch.equal(getattr(graphed, f), getattr(eager, f)), (t, f)
        # resident slots only: a dropped prediction's slot is empty, and how much of it the
        # live copy wrote before stopping depends on timing
        live = graphed.slot_expert >= 0
        for n in NAMES:
            assert torch.equal(graphed.slots[n][live], eager.slots[n][live]), (t, n)
        _all_slots_hold_their_experts(graphed, src)


def test_cache_prefetch_edge_cases(monkeypatch):
    """Two prefetches in a row (the second waits for the first copy), a budget of one
    install, an over-long prediction (refused, nothing launched), and join() with nothing
    pending."""
    monkeypatch.setenv("EXPERT_CACHE_POLICY", "lfu")
    monkeypatch.setenv("EXPERT_CACHE_DECAY", "64")
    owner = Owner(4)
    src = _device_sources(owner)
    cache = ExpertSlotCache(owner, NAMES, E, S, gu.DEV)
    ref = oracle.State(E, S)
    cache.join()
    rng = np.random.default_rng(31)
    for t in range(30):
        ids = rng.choice(E, K, replace=False).astype(np.int32)
        p1 = rng.choice(E, K, replace=False).astype(np.int32)
        p2 = _predict(ids, E, 0.5, rng).astype(np.int32)
        assert cache.prefetch(torch.as_tensor(p1, device=gu.DEV))
        assert cache.prefetch(torch.as_tensor(p2, device=gu.DEV), max_inserts=1)
        assert not cache.prefetch(torch.zeros(S + 1, dtype=torch.int32, device=gu.DEV))
        slot_ids = cache.refresh(torch.as_tensor(ids, device=gu.DEV))
        assert ref.prefetch(p1, S) == 0
        assert ref.prefetch(p2, 1) == 0
        assert ref.n_miss[0] <= 1
        assert ref.manage(ids, K, S, 1, 64) == 0
        torch.cuda.synchronize()
        assert np.array_equal(slot_ids.cpu().numpy(), oracle.remap(ids, ref.table)), t
        for f in ("table", "slot_expert", "slot_stamp", "step"):
            assert np.array_equal(getattr(cache, f).cpu().numpy(), getattr(ref, f)), (t, f)
        _all_slots_hold_their_experts(cache, src)


def test_two_layer_pipeline_shares_the_side_stream():
    """The plugin's order over two layers: layer 1's prefetch is issued while layer 0
    refreshes, through the one side stream; every resident slot of both layers holds its
    expert's bytes after each step."""
    owners = [Owner(5), Owner(6)]
    srcs = [_device_sources(o) for o in owners]
    caches = [ExpertSlotCache(o, NAMES, E, S, gu.DEV) for o in owners]
    rng = np.random.default_rng(41)
    busy = torch.randn((1024, 1024), device=gu.DEV)
    nxt0 = rng.choice(E, K, replace=False).astype(np.int32)
    for t in range(40):
        ids0 = nxt0
        ids1 = rng.choice(E, K, replace=False).astype(np.int32)
        nxt0 = rng.choice(E, K, replace=False).astype(np.int32)
        assert caches[1].prefetch(torch.as_tensor(_predict(ids1, E, 0.75, rng), device=gu.DEV))
        s0 = caches[0].refresh(torch.as_tensor(ids0, device=gu.DEV))
        t0 = caches[0].table.clone()  # the table the step's slot ids refer to
        busy = busy @ busy.T * 1e-3
        s1 = caches[1].refresh(torch.as_tensor(ids1, device=gu.DEV))
        t1 = caches[1].table.clone()
        # the next step's prefetch for layer 0 may evict this step's experts: it is ordered
        # after everything already queued on the stream
        assert caches[0].prefetch(torch.as_tensor(nxt0, device=gu.DEV))
        torch.cuda.synchronize()
        for c, src in zip(caches, srcs):
            _all_slots_hold_their_experts(c, src)
        for table, ids, out in ((t0, ids0, s0), (t1, ids1, s1)):
            table = table.cpu().numpy()
            assert np.array_equal(out.cpu().numpy(), table[ids]), t
            assert (table[ids] >= 0).all()
    caches[0].join()
    torch.cuda.synchronize()
    _all_slots_hold_their_experts(caches[0], srcs[0])
