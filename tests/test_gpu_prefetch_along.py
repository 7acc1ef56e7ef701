"""One launch for two layers: expert_cache_manage_remap_prefetch against the oracle, and
ExpertSlotCache.prefetch(..., along=) against the same calls made one at a time.

Kernel parity: two layers' states sit in adjacent rows of one allocation (so the host's
overlap check must accept arrays that touch without overlapping). Step t runs layer
t % 2's policy step and remap and the other layer's prefetch of its next routing in one
launch, so each layer alternates prefetch -> manage, the plugin's order. After every launch
both layers' miss lists, prefetch miss lists, slot ids and full state must equal the
oracle's, bit for bit. The cases reach every launch variant (slots per lane 1-16, table
chunks 1-8, experts beyond the LDS table), int32 and int64 routing ids, insert budgets of
0, 1 and S, and predictions that are right, partly wrong or all wrong.

Cache level: a two-layer decode with the prefetch staged along the other layer's refresh
leaves states, slot ids and slot bytes equal to the same decode with the prefetch launched
on its own, eagerly and in graph replays; staged steps are launched on their own when the
carrying layer is joined (the read-through branch), refreshed out of order, or restaged.
"""
from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle
from test_gpu_cache import NAMES, Owner
from test_gpu_prefetch import _initial_stamps, _predict, _routing, _words
from vllm_expert_cache.cache import ExpertSlotCache

pytestmark = pytest.mark.gpu

LRU, LFU = 0, 1

# name, E, S, mk, prefetch budget, policy, decay, accuracy, initial stamps, id bytes
CASES = [
    ("e128-s64", 128, 64, 8, 64, LFU, 64, 0.8, None, 4),
    ("e128-s64-lru-i64", 128, 64, 8, 64, LRU, 64, 1.0, None, 8),
    ("e8-s4", 8, 4, 2, 4, LFU, 64, 0.5, None, 4),
    ("e256-s128-i64", 256, 128, 128, 128, LFU, 64, 0.7, None, 8),
    ("e512-s257", 512, 257, 50, 64, LRU, 0, 0.6, None, 4),
    ("e1000-s1024", 1000, 1024, 200, 1024, LFU, 3, 0.5, None, 4),
    ("e5000-s300", 5000, 300, 64, 300, LRU, 0, 0.6, None, 8),
    ("e128-s16-budget1", 128, 16, 8, 1, LFU, 64, 0.7, None, 4),
    ("e128-s16-budget0", 128, 16, 8, 0, LRU, 64, 0.7, None, 4),
    ("e257-s65-wide", 257, 65, 64, 65, LFU, 64, 0.0, "wide", 4),
    ("e64-s129-neg", 64, 129, 33, 129, LFU, 0, 0.5, "neg", 4),
]


def _oracle_prefetch(ref: oracle.State, pred, budget, pf):
    """ref.prefetch into the prefetch miss list `pf` = (miss, n_miss), keeping ref's own."""
    keep = ref.miss.copy(), ref.n_miss.copy()
    ref.miss[:], ref.n_miss[:] = pf
    assert ref.prefetch(pred, budget) == 0
    out = ref.miss.copy(), ref.n_miss.copy()
    ref.miss[:], ref.n_miss[:] = keep
    return out


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_one_launch_matches_oracle(case):
    name, E, S, mk, budget, policy, decay, acc, stamps, idb = case
    T = 160
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    ids = _routing(E, mk, T + 1, rng)
    pred = _predict(ids, E, acc, rng)
    init = [_initial_stamps(stamps, S, rng) for _ in range(2)]
    cap = max(S, budget, 1)
    print(f"case {name}: E={E} S={S} mk={mk} budget={budget} acc={acc} ids int{8 * idb}",
          flush=True)

    h = gu.lib()
    st = gu.Layers(2, E, S, miss_cap=cap)
    for l in range(2):
        if init[l] is not None:
            st.slot_stamp[l].copy_(torch.as_tensor(init[l], device=gu.DEV))
    pf_miss = torch.zeros((2, 2 * cap), dtype=torch.int32, device=gu.DEV)
    pf_n = torch.zeros((2, 1), dtype=torch.int32, device=gu.DEV)
    d_ids = torch.as_tensor(ids.astype(np.int64 if idb == 8 else np.int32), device=gu.DEV)
    d_pred = torch.as_tensor(pred, device=gu.DEV)
    out = torch.full((T, mk), -9, dtype=d_ids.dtype, device=gu.DEV)
    words = oracle.state_words(E, S)
    rec = {k: torch.zeros(shape, dtype=torch.int32, device=gu.DEV) for k, shape in (
        ("n", (T, 2)), ("miss", (T, 2, 2 * cap)), ("pf_n", (T, 2)),
        ("pf_miss", (T, 2, 2 * cap)), ("state", (T, 2, words)))}
    md = min(E, mk)

    def row(t, l):
        return gu.P(t.data_ptr() + l * t.stride(0) * t.element_size())

    # layer 1's first prefetch on its own, then the pairs
    assert h.expert_cache_prefetch(row(d_pred, 0), mk, E, S, budget, st.row("table", 1),
                                   st.row("map_cold", 1), st.row("slot_expert", 1),
                                   st.row("slot_stamp", 1), st.row("routed", 1),
                                   row(pf_miss, 1), row(pf_n, 1), gu.stream()) == 0
    for t in range(T):
        j, k = t % 2, 1 - t % 2
        rc = h.expert_cache_manage_remap_prefetch(
            row(d_ids, t), idb, mk, E, S, md, S, st.row("table", j), st.row("map_cold", j),
            st.row("slot_expert", j), st.row("slot_stamp", j), st.row("routed", j),
            st.row("step", j), st.row("miss", j), st.row("n_miss", j), policy, decay,
            row(out, t), row(d_pred, t + 1), mk, budget, st.row("table", k),
            st.row("map_cold", k), st.row("slot_expert", k), st.row("slot_stamp", k),
            st.row("routed", k), row(pf_miss, k), row(pf_n, k), gu.stream())
        assert rc == 0, rc
        rec["n"][t].copy_(st.n_miss[:, 0])
        rec["miss"][t].copy_(st.miss)
        rec["pf_n"][t].copy_(pf_n[:, 0])
        rec["pf_miss"][t].copy_(pf_miss)
        rec["state"][t].copy_(st.state_words())
    torch.cuda.synchronize()
    got = {k: v.cpu().numpy() for k, v in rec.items()}
    got_out = out.cpu().numpy()

    refs = [oracle.State(E, S, miss_cap=cap) for _ in range(2)]
    for l in range(2):
        if init[l] is not None:
            refs[l].slot_stamp[:] = init[l]
    pf = [(np.zeros(2 * cap, np.int32), np.zeros(1, np.int32)) for _ in range(2)]
    pf[1] = _oracle_prefetch(refs[1], pred[0], budget, pf[1])
    want = {k: np.zeros_like(v) for k, v in got.items()}
    want_out = np.zeros_like(got_out)
    for t in range(T):
        j, k = t % 2, 1 - t % 2
        assert refs[j].manage(ids[t], md, S, policy, decay) == 0
        want_out[t] = oracle.remap(ids[t], refs[j].table)
        pf[k] = _oracle_prefetch(refs[k], pred[t + 1], budget, pf[k])
        for l in range(2):
            want["n"][t, l] = refs[l].n_miss[0]
            want["miss"][t, l] = refs[l].miss
            want["pf_n"][t, l] = pf[l][1][0]
            want["pf_miss"][t, l] = pf[l][0]
            want["state"][t, l] = _words(refs[l])

    for k in ("n", "miss", "pf_n", "pf_miss", "state"):
        d = gu.first_diff(got[k], want[k])
        assert d is None, f"{name}: {k} differs first at {d}: {got[k][d]} != {want[k][d]}"
    d = gu.first_diff(got_out, want_out)
    assert d is None, f"{name}: slot ids differ first at {d}"
    print(f"  prefetched {int(want['pf_n'].sum())}, real inserts {int(want['n'].sum())}",
          flush=True)


E, S, K = 128, 32, 8


def _sources(owner):
    return {n: getattr(owner, n).to(gu.DEV) for n in NAMES}


def _holds(cache: ExpertSlotCache, src: dict):
    live = torch.nonzero(cache.slot_expert >= 0).flatten()
    experts = cache.slot_expert[live].long()
    for n in NAMES:
        assert torch.equal(cache.slots[n][live], src[n][experts]), n


FIELDS = ("table", "map_cold", "slot_expert", "slot_stamp", "step", "miss", "n_miss",
          "pf_miss", "pf_n_miss")


def _same(a: ExpertSlotCache, b: ExpertSlotCache, t):
    """Every state field, and the bytes of every resident slot (a dropped prediction's slot
    is empty, and how much of it the live copy wrote before stopping depends on timing)."""
    for f in FIELDS:
        assert torch.equal(getattr(a, f), getattr(b, f)), (t, f)
    live = a.slot_expert >= 0
    for n in NAMES:
        assert torch.equal(a.slots[n][live], b.slots[n][live]), (t, n)


def _pair(seed):
    """Two layers' caches, slot bytes zeroed."""
    owners = [Owner(seed), Owner(seed + 1)]
    caches = [ExpertSlotCache(o, NAMES, E, S, gu.DEV) for o in owners]
    for c in caches:
        for buf in c.slots.values():
            buf.zero_()
    return owners, caches


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_cache_along_equals_separate_launches(dtype):
    """Two-layer decode: layer 1's prefetch staged along layer 0's refresh, and layer 0's
    next-step prefetch staged on layer 1, against the same prefetches launched on their
    own. Some steps also restage (the first staged step then runs alone) or read layer 0
    through (join launches what is staged on it and what it has staged elsewhere). Routing
    ids and predictions come as int32 or int64, as vLLM may hand either."""
    owners, along = _pair(11)
    _, alone = _pair(11)
    srcs = [_sources(o) for o in owners]
    rng = np.random.default_rng(51)
    busy = torch.randn((1024, 1024), device=gu.DEV)
    nxt0 = rng.choice(E, K, replace=False).astype(np.int32)
    for t in range(48):
        ids0 = nxt0
        ids1 = rng.choice(E, K, replace=False).astype(np.int32)
        nxt0 = rng.choice(E, K, replace=False).astype(np.int32)
        p1 = torch.as_tensor(_predict(ids1, E, 0.75, rng), device=gu.DEV).to(dtype)
        p1b = torch.as_tensor(rng.choice(E, 4, replace=False).astype(np.int32),
                              device=gu.DEV).to(dtype)
        p0 = torch.as_tensor(_predict(nxt0, E, 0.75, rng), device=gu.DEV).to(dtype)
        d0 = torch.as_tensor(ids0, device=gu.DEV).to(dtype)
        d1 = torch.as_tensor(ids1, device=gu.DEV).to(dtype)
        mode = t % 4
        # with along=
        if mode == 1:  # restaged: the first prediction runs alone, the second rides
            assert along[1].prefetch(p1b, max_inserts=2, along=along[0])
        assert along[1].prefetch(p1, along=along[0])
        if mode == 3:  # layer 0 read through: join launches the staged step on its own
            along[0].join()
            assert along[0]._rider is None and along[1]._riding_on is None
        else:
            s0a = along[0].refresh(d0)
        busy = busy @ busy.T * 1e-3
        s1a = along[1].refresh(d1)
        # the same, each prefetch launched where it was staged
        if mode == 1:
            assert alone[1].prefetch(p1b, max_inserts=2)
        assert alone[1].prefetch(p1)
        if mode == 3:
            alone[0].join()
        else:
            s0b = alone[0].refresh(d0)
        s1b = alone[1].refresh(d1)
        torch.cuda.synchronize()
        if mode != 3:
            assert torch.equal(s0a, s0b), t
        assert torch.equal(s1a, s1b), t
        for a, b, src in zip(along, alone, srcs):
            _same(a, b, t)
            _holds(a, src)
        # layer 0's next prediction: staged on layer 1, which has no refresh before layer
        # 0's, so layer 0's refresh (or join) launches it on its own first
        assert along[0].prefetch(p0, along=along[1])
        assert alone[0].prefetch(p0)


def test_cache_along_under_graph_capture():
    """A captured two-layer step with both prefetches staged along the other layer's
    refresh, replayed against an eager twin running the same calls."""
    owners, graphed = _pair(21)
    _, eager = _pair(21)
    srcs = [_sources(o) for o in owners]
    rng = np.random.default_rng(61)
    ids = [torch.zeros((2, K), dtype=torch.int32, device=gu.DEV) for _ in range(2)]
    pred = [torch.zeros((2, K), dtype=torch.int32, device=gu.DEV) for _ in range(2)]

    def step(c, ids, pred):
        c[1].prefetch(pred[1], along=c[0])
        o0 = c[0].refresh(ids[0])
        o1 = c[1].refresh(ids[1])
        c[0].prefetch(pred[0])
        return o0, o1

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step(graphed, ids, pred)
        step(eager, ids, pred)
        for c in graphed + eager:
            c.join()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = step(graphed, ids, pred)
        graphed[0].join()
    for t in range(40):
        for l in range(2):
            r = np.stack([rng.choice(E, K, replace=False) for _ in range(2)]).astype(np.int32)
            ids[l].copy_(torch.as_tensor(r, device=gu.DEV))
            pred[l].copy_(torch.as_tensor(_predict(r, E, 0.6, rng), device=gu.DEV))
        g.replay()
        want = step(eager, [i.clone() for i in ids], [p.clone() for p in pred])
        eager[0].join()
        torch.cuda.synchronize()
        for a, b in zip(outs, want):
            assert torch.equal(a, b), t
        for a, b, src in zip(graphed, eager, srcs):
            _same(a, b, t)
            _holds(a, src)


def test_cache_along_refuses_bad_partners():
    owners, caches = _pair(31)
    other = ExpertSlotCache(Owner(40), NAMES, E, S // 2, gu.DEV)
    pred = torch.zeros(K, dtype=torch.int32, device=gu.DEV)
    with pytest.raises(ValueError):
        caches[0].prefetch(pred, along=caches[0])
    with pytest.raises(ValueError):
        caches[0].prefetch(pred, along=other)
    # wider than the slots: refused before anything is staged
    assert not caches[0].prefetch(torch.zeros(S + 1, dtype=torch.int32, device=gu.DEV),
                                  along=caches[1])
    assert caches[1]._rider is None
    # refreshing the staged layer first launches its staged step on its own
    assert caches[1].prefetch(pred, along=caches[0])
    caches[1].refresh(torch.arange(K, dtype=torch.int32, device=gu.DEV))
    assert caches[0]._rider is None and caches[1]._riding_on is None
    torch.cuda.synchronize()
    for c, o in zip(caches, owners):
        _holds(c, _sources(o))
