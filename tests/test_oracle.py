"""Pins for the CPU oracle (oracle/policy.c), before the GPU results are checked against it.

  * Known answers: the reference's 12 published insert counts (README.md:177-184) on its
    own harness's traces (tests/compare_policies.py:31-93), regenerated with numpy.
  * Two independent victim rules -- serial argmin per insert (tests/test_policy.py:117-131)
    and batched rank-select (kernels/expert_cache.hip:159-188) -- must agree on every field
    of every step, on every routing pattern the reference's suites use.
  * Hand-worked steps that pin each rule of the step: ascending-id miss order, (stamp, slot)
    victim order, the never-evict-what-is-routed rule, LFU +1 before halving, no ageing on
    a step without inserts, the insert cap and its miss-buffer side effect, read-through,
    padding ids.
  * Invariants after every step (tests/test_policy.py:162-169).
"""
from __future__ import annotations

import numpy as np
import pytest

import kat_traces
import oracle
from oracle import State

LRU, LFU = 0, 1


# ---- known answers ----------------------------------------------------------------------

@pytest.mark.parametrize("rule", ["rank", "serial"])
@pytest.mark.parametrize("key", sorted(kat_traces.KAT))
def test_published_insert_counts(key, rule):
    workload, slots = key
    trace = kat_traces.trace(workload)
    assert trace.shape == (kat_traces.STEPS, kat_traces.TOP_K)
    want_lru, want_lfu = kat_traces.KAT[key]
    got_lru = oracle.run_trace(trace, kat_traces.E, slots, LRU, 64, rule)["n_miss"].sum()
    got_lfu = oracle.run_trace(trace, kat_traces.E, slots, LFU, 64, rule)["n_miss"].sum()
    assert (got_lru, got_lfu) == (want_lru, want_lfu)


def test_known_answers_detect_a_wrong_rule():
    """The counts are sensitive enough to catch plausible slips: ageing on every step,
    or evicting the highest key instead of the lowest, changes them."""
    trace = kat_traces.trace("zipf")
    base = oracle.run_trace(trace, 128, 32, LFU, 64)["n_miss"].sum()
    assert base == kat_traces.KAT[("zipf", 32)][1]
    assert oracle.run_trace(trace, 128, 32, LFU, 1)["n_miss"].sum() != base
    assert oracle.run_trace(trace, 128, 32, LFU, 0)["n_miss"].sum() != base


# ---- hand-worked steps --------------------------------------------------------------------

def _step(st: State, ids, policy, decay=64, md=None, mi=None, rule="rank"):
    ids = np.asarray(ids, dtype=np.int32)
    md = min(st.E, ids.size) if md is None else md
    mi = st.S if mi is None else mi
    assert st.manage(ids, md, mi, policy, decay, rule) == 0


@pytest.mark.parametrize("rule", ["rank", "serial"])
def test_lru_hand_worked(rule):
    st = State(6, 3)
    _step(st, [4, 1], LRU, rule=rule)          # misses in id order: 1 -> slot 0, 4 -> slot 1
    assert st.misses() == [(1, 0), (4, 1)]
    assert st.table.tolist() == [-1, 0, -1, -1, 1, -1]
    assert st.map_cold.tolist() == [0, -1, 2, 3, -1, 5]
    assert st.slot_stamp.tolist() == [1, 1, 0]
    _step(st, [1, 5], LRU, rule=rule)          # 1 hits; the empty slot 2 has the lowest key
    assert st.misses() == [(5, 2)]
    assert st.slot_expert.tolist() == [1, 4, 5]
    assert st.slot_stamp.tolist() == [2, 1, 2]
    _step(st, [0, 2], LRU, rule=rule)          # keys: slot1 (1,1) < slot0 (2,0) < slot2 (2,2)
    assert st.misses() == [(0, 1), (2, 0)]
    assert st.slot_expert.tolist() == [2, 0, 5]
    assert st.table.tolist() == [1, -1, 0, -1, -1, 2]
    assert st.map_cold.tolist() == [-1, 1, -1, 3, 4, -1]
    assert st.slot_stamp.tolist() == [3, 3, 2]
    _step(st, [2, 2], LRU, rule=rule)          # duplicate id, a pure hit: nothing inserted
    assert st.n_miss[0] == 0
    assert st.slot_stamp.tolist() == [4, 3, 2]
    assert st.miss[:4].tolist() == [0, 1, 2, 0]  # miss buffer left as it was
    assert st.step[0] == 4
    assert st.routed.tolist() == [0, 0, 1, 0, 0, 0]


@pytest.mark.parametrize("rule", ["rank", "serial"])
def test_lfu_decay_hand_worked(rule):
    st = State(6, 2)
    _step(st, [3, 1], LFU, decay=2, rule=rule)  # installs start at count 1
    assert st.slot_expert.tolist() == [1, 3] and st.slot_stamp.tolist() == [1, 1]
    _step(st, [1, 3], LFU, decay=2, rule=rule)  # step 2 is a decay step, but no insert:
    assert st.slot_stamp.tolist() == [2, 2]     # counts grow and nothing halves
    _step(st, [1, 4], LFU, decay=2, rule=rule)
    assert st.misses() == [(4, 1)] and st.slot_stamp.tolist() == [3, 1]
    _step(st, [1, 5], LFU, decay=2, rule=rule)  # +1 (3 -> 4) lands before the halving (-> 2)
    assert st.misses() == [(5, 1)] and st.slot_stamp.tolist() == [2, 1]
    _step(st, [2, 5], LFU, decay=2, rule=rule)  # 5 hits (1 -> 2); 2 evicts expert 1
    assert st.misses() == [(2, 0)]
    assert st.slot_expert.tolist() == [2, 5] and st.slot_stamp.tolist() == [1, 2]


@pytest.mark.parametrize("rule", ["rank", "serial"])
def test_insert_cap_and_miss_buffer(rule):
    st = State(8, 2, miss_cap=3)
    st.miss[:] = -7
    _step(st, [0, 1, 2, 3], LRU, md=8, mi=3, rule=rule)
    # three inserts allowed, only two slots: the third expert is listed but not placed
    assert st.n_miss[0] == 2
    assert st.miss.tolist() == [0, 0, 1, 1, 2, -7]
    assert st.table.tolist() == [0, 1, -1, -1, -1, -1, -1, -1]


@pytest.mark.parametrize("rule", ["rank", "serial"])
def test_never_evicts_a_routed_expert(rule):
    st = State(8, 2)
    _step(st, [0, 1], LRU, rule=rule)
    _step(st, [0, 1, 2], LRU, md=8, mi=2, rule=rule)  # both slots routed: no victim
    assert st.n_miss[0] == 0
    assert st.miss[0] == 2                          # listed before the search came up empty
    assert st.slot_expert.tolist() == [0, 1] and st.slot_stamp.tolist() == [2, 2]


@pytest.mark.parametrize("rule", ["rank", "serial"])
def test_read_through_changes_only_step_and_flags(rule):
    st = State(8, 4)
    _step(st, [5, 6], LRU, rule=rule)
    before = st.copy()
    _step(st, [0, 1, 2], LRU, md=2, rule=rule)
    assert st.step[0] == 2 and st.n_miss[0] == 0
    assert st.routed.tolist() == [1, 1, 1, 0, 0, 0, 0, 0]
    for f in ("table", "map_cold", "slot_expert", "slot_stamp", "miss"):
        assert np.array_equal(getattr(st, f), getattr(before, f)), f


@pytest.mark.parametrize("rule", ["rank", "serial"])
def test_padding_ids_are_ignored(rule):
    st = State(8, 4)
    _step(st, [-1, 7, 9, -5], LRU, md=4, rule=rule)
    assert st.misses() == [(7, 0)]
    assert st.routed.tolist() == [0] * 7 + [1]


def test_bad_arguments_rejected():
    st = State(8, 4)
    for E, S, mi, pol in ((0, 4, 4, 0), (8, 0, 4, 0), (8, 1025, 4, 0), (8, 4, -1, 0),
                          (8, 4, 1025, 0), (8, 4, 4, 2), (8, 4, 4, -1)):
        st.E, st.S = E, S
        assert st.manage([1], 1, mi, pol, 64) == -1
    assert st.step[0] == 0  # a rejected call changes nothing


# ---- serial rule == rank rule, every field, every step ------------------------------------

def _suite_traces():
    """Routing of the reference's policy suites (tests/test_policy.py:202-221), generated
    with our own seeds; each entry: name, E, S, ids[T, mk], max_distinct, max_inserts."""
    rng = np.random.default_rng(0)
    zipf = np.arange(1, 513, dtype=float) ** -1.1
    zipf /= zipf.sum()
    padded = rng.choice(64, size=(120, 4, 10))
    padded[:, 2:] = -1
    return [
        ("tiny-churn", 32, 8, rng.choice(32, size=(200, 10)), 8, 8),
        ("skewed-512", 512, 257, np.stack([np.concatenate(
            [rng.choice(512, 10, replace=False, p=zipf) for _ in range(5)])
            for _ in range(120)]), 128, 64),
        ("insert-capped", 128, 32, rng.choice(128, size=(150, 80)), 128, 4),
        ("read-through", 128, 32, rng.choice(128, size=(60, 160)), 8, 16),
        ("padded-rows", 64, 16, padded.reshape(120, 40), 64, 16),
    ]


@pytest.mark.parametrize("policy", [LRU, LFU])
@pytest.mark.parametrize("suite", _suite_traces(), ids=lambda s: s[0])
def test_serial_equals_rank_on_reference_suites(suite, policy):
    name, E, S, ids, md, mi = suite
    rng = np.random.default_rng(1)
    hot = sorted(rng.choice(E, S, replace=False).tolist())  # warm start, stamp 0
    a, b = State(E, S, hot, miss_cap=mi), State(E, S, hot, miss_cap=mi)
    for t in range(ids.shape[0]):
        assert a.manage(ids[t], md, mi, policy, 8, "serial") == 0
        assert b.manage(ids[t], md, mi, policy, 8, "rank") == 0
        for f in State.FIELDS:
            assert np.array_equal(getattr(a, f), getattr(b, f)), (name, t, f)
        _check_invariants(b)


@pytest.mark.parametrize("policy", [LRU, LFU])
@pytest.mark.parametrize("slots", [16, 64])
def test_serial_equals_rank_on_synthetic_trace(policy, slots):
    from vllm_expert_cache import traces

    w = traces.WORKLOADS["single-layer-e128"]
    ids = traces.routing(w, 0, steps=1500)
    a = oracle.run_trace(ids, 128, slots, policy, 64, "serial", record_miss=True,
                         record_state=True)
    b = oracle.run_trace(ids, 128, slots, policy, 64, "rank", record_miss=True,
                         record_state=True)
    for k in ("n_miss", "miss", "state"):
        assert np.array_equal(a[k], b[k]), k


def _check_invariants(s: State):
    t, c, se = s.table, s.map_cold, s.slot_expert
    # table and map_cold are complementary
    assert (((t >= 0) & (c == -1)) | ((t < 0) & (c == np.arange(s.E)))).all()
    live = se[se >= 0]
    assert len(np.unique(live)) == len(live)                 # no expert in two slots
    assert (t[live] == np.nonzero(se >= 0)[0]).all()          # table[slot_expert[s]] == s
    assert (t >= 0).sum() == len(live)


@pytest.mark.parametrize("policy", [LRU, LFU])
def test_every_routed_id_resident_after_a_served_step(policy):
    from vllm_expert_cache import traces

    w = traces.WORKLOADS["48-layer-e128-batch4"]
    ids = traces.routing(w, 3, steps=300)
    st = State(128, 32)
    for t in range(ids.shape[0]):
        assert st.manage(ids[t], min(128, ids.shape[1]), 32, policy, 64) == 0
        routed = np.unique(ids[t])
        assert (st.table[routed] >= 0).all()
        assert st.n_miss[0] == len(st.misses())
        _check_invariants(st)


# ---- remap / gather / fused ----------------------------------------------------------------

@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_remap_matches_numpy_indexing(dtype):
    rng = np.random.default_rng(5)
    table = rng.integers(-1, 64, size=128).astype(np.int32)
    ids = rng.integers(-128, 128, size=1000).astype(dtype)   # includes negative wrap
    got = oracle.remap(ids, table)
    assert got.dtype == dtype
    assert np.array_equal(got, table[ids].astype(dtype))     # numpy wraps like torch
    bad = np.array([128, -129, 1 << 20], dtype=dtype)
    assert oracle.remap(bad, table).tolist() == [-1, -1, -1]


def test_gather_matches_slicing():
    rng = np.random.default_rng(6)
    E, S, sizes = 10, 4, [48, 16, 160]
    src = [rng.integers(0, 256, size=E * b, dtype=np.uint8) for b in sizes]
    dst = [np.zeros(S * b, np.uint8) for b in sizes]
    miss = np.array([7, 2, 3, 0, 9, 3], np.int32)
    oracle.gather(dst, src, sizes, miss, 2)  # only the first two pairs
    for d, s, b in zip(dst, src, sizes):
        assert np.array_equal(d[2 * b:3 * b], s[7 * b:8 * b])
        assert np.array_equal(d[0:b], s[3 * b:4 * b])
        assert not d[3 * b:].any() and not d[b:2 * b].any()


def _align_brute(ids, table, E, S, bs, L, NB):
    """moe_align_block_size for both sides, by sorting (bucket, token) pairs."""
    out = {}
    for side in ("hot", "cold"):
        pairs = []
        for i, e in enumerate(ids):
            if not 0 <= e < E:
                continue
            s = table[e]
            hot = 0 <= s < S
            if (side == "hot") == hot:
                pairs.append((s if hot else e, i))
        pairs.sort()
        sorted_ids = np.full(L, len(ids), np.int32)
        eids = np.full(NB, -1, np.int32)
        pos = 0
        nb = S if side == "hot" else E
        for b in range(nb):
            toks = [i for (k, i) in pairs if k == b]
            if not toks:
                continue
            sorted_ids[pos:pos + len(toks)] = toks
            padded = -(-len(toks) // bs) * bs
            eids[pos // bs:(pos + padded) // bs] = b
            pos += padded
        out[f"sorted_{side}"] = sorted_ids
        out[f"eids_{side}"] = eids
        out[f"npad_{side}"] = np.array([pos], np.int32)
    return out


def align_lengths(mk, E, bs):
    """vLLM's buffer lengths (kernels/expert_cache.hip:606-609)."""
    L = min(mk * bs, mk + E * (bs - 1)) if mk < E else mk + E * (bs - 1)
    return L, -(-L // bs)


@pytest.mark.parametrize("bs", [1, 4, 16])
def test_fused_matches_brute_force_align(bs):
    from vllm_expert_cache import traces

    w = traces.WORKLOADS["48-layer-e128-batch4"]
    ids = traces.routing(w, 1, steps=80)
    E, S = 128, 48
    mk = ids.shape[1]
    L, NB = align_lengths(mk, E, bs)
    st, ref = State(E, S), State(E, S)
    for t in range(ids.shape[0]):
        row = ids[t].copy()
        row[::7] = -1                                    # some padding ids
        rc, got = st.fused(row, min(E, mk), S, bs, L, NB)
        assert rc == 0
        assert ref.manage(row, min(E, mk), S, LRU, 0) == 0   # fused = LRU manage, no decay
        for f in State.FIELDS:
            assert np.array_equal(getattr(st, f), getattr(ref, f)), (t, f)
        want = _align_brute(row.tolist(), st.table, E, S, bs, L, NB)
        for k, v in want.items():
            assert np.array_equal(got[k], v), (t, k)


@pytest.mark.parametrize("seed", range(60))
def test_serial_equals_rank_on_random_shapes(seed):
    """The GPU fuzz's shape and argument space (tests/test_gpu_fuzz.py), both oracle forms."""
    rng = np.random.default_rng(1000 + seed)
    E = int(rng.choice([1, 2, 7, 64, 128, 257, 1000, 4100]))
    S = int(rng.choice([1, 2, 3, 16, 64, 65, 129, 300, 1024]))
    mk = int(rng.choice([0, 1, 8, 33, 257, 700]))
    mi = int(rng.choice([0, 1, 4, S, 1024]))
    policy, decay = int(rng.integers(0, 2)), int(rng.choice([0, 1, 3, 64]))
    nhot = int(rng.integers(0, min(S, E) + 1))
    hot, slots = rng.choice(E, nhot, replace=False), rng.choice(S, nhot, replace=False)
    a, b = State(E, S, miss_cap=max(mi, 1)), State(E, S, miss_cap=max(mi, 1))
    for st in (a, b):
        st.table[hot] = slots
        st.map_cold[hot] = -1
        st.slot_expert[slots] = hot
        st.slot_stamp[:] = rng.integers(0, 1000, size=S) if st is a else a.slot_stamp
    for t in range(10):
        ids = rng.integers(-3, E + 3, size=mk).astype(np.int32)
        md = int(rng.choice([E, mk, -1, len(np.unique(ids[(ids >= 0) & (ids < E)])) - 1]))
        assert a.manage(ids, md, mi, policy, decay, "serial") == 0
        assert b.manage(ids, md, mi, policy, decay, "rank") == 0
        for f in State.FIELDS:
            assert np.array_equal(getattr(a, f), getattr(b, f)), (seed, t, f)
        _check_invariants(b)


def test_fused_trace_is_the_stepwise_fused():
    """oracle_fused_trace (bench.py's CPU timing loop) leaves the state that calling the
    fused step once per row leaves."""
    from vllm_expert_cache import traces

    w = traces.WORKLOADS["48-layer-e128-batch4"]
    ids = traces.routing(w, 2, steps=60)
    E, S, bs = 128, 48, 16
    mk = ids.shape[1]
    L, NB = align_lengths(mk, E, bs)
    a, b = State(E, S), State(E, S)
    for row in ids:
        rc, _ = a.fused(row, min(E, mk), S, bs, L, NB)
        assert rc == 0
    assert b.fused_trace(ids, bs, L, NB) == 0
    for f in ("table", "map_cold", "slot_expert", "slot_stamp", "step", "miss", "n_miss"):
        assert np.array_equal(getattr(a, f), getattr(b, f)), f
