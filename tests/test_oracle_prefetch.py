"""Pins for the oracle's prefetch step (oracle/policy.c, `oracle_prefetch`).

The reference names next-layer prefetch (README.md:392-394) but does not implement it, so
the step's rules are this library's own. They are pinned here against the already-pinned
manage rules rather than against a restatement of themselves:

  * A right prediction changes nothing the policy can see: prefetch(R) followed by
    manage(R) leaves every field equal to manage(R) alone, with the miss list moved to
    the prefetch, on every step that would not age the LFU counts (a dropped stamp-0
    install, a hit counted twice, a moved step counter or a different victim all break it).
  * A wrong prediction leaves nothing behind: prefetch(P) followed by manage(R), with P
    disjoint from R, equals manage(R) on the state the prefetch left with the predicted
    experts' slots emptied (stamp 0), i.e. the only trace of the prediction is what it
    evicted.
  * Two independent victim rules (serial argmin, rank) agree on every field.
  * Hand-worked steps for the pending marker (install stamp -1; the next served step
    confirms or drops, after any ageing, once), an all-resident prediction, a zero budget,
    and invariants after wrong predictions.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from oracle import State
from test_oracle import _check_invariants

LRU, LFU = 0, 1
POLICY_FIELDS = ("table", "map_cold", "slot_expert", "slot_stamp", "routed", "step")


def test_hand_worked_prefetch():
    st = State(8, 4)
    st.slot_expert[:] = [0, 1, 2, -1]
    st.slot_stamp[:] = [5, 2, 7, 0]
    st.table[:3] = [0, 1, 2]
    st.map_cold[:3] = -1
    st.step[0] = 9
    assert st.prefetch([3, 1, 5, 99, -2], max_inserts=4) == 0
    # routed {1, 3, 5}; 1 is resident and keeps stamp 2; misses 3, 5 in id order take the
    # two lowest keys among slots not predicted: slot 3 (0, 3) then slot 0 (5, 0); both
    # installs are pending (stamp -1)
    assert st.misses() == [(3, 3), (5, 0)]
    assert st.slot_expert.tolist() == [5, 1, 2, 3]
    assert st.slot_stamp.tolist() == [-1, 2, 7, -1]
    assert st.table.tolist() == [-1, 1, 2, 3, -1, 0, -1, -1]
    assert st.map_cold.tolist() == [0, -1, -1, -1, 4, -1, 6, 7]
    assert st.routed.tolist() == [0, 1, 0, 1, 0, 1, 0, 0]
    assert st.step[0] == 9


@pytest.mark.parametrize("rule", ["rank", "serial"])
def test_resident_prediction_and_zero_budget_change_nothing(rule):
    rng = np.random.default_rng(5)
    st = State(64, 16, hot=sorted(rng.choice(64, 16, replace=False).tolist()))
    st.slot_stamp[:] = rng.integers(0, 50, 16)
    st.step[0] = 77
    st.n_miss[0] = 3
    before = st.copy()
    assert st.prefetch(st.slot_expert[[2, 5, 5, 9]], st.S, rule) == 0
    assert st.n_miss[0] == 0
    for f in ("table", "map_cold", "slot_expert", "slot_stamp", "step"):
        assert np.array_equal(getattr(st, f), getattr(before, f)), f
    cold = np.nonzero(st.table < 0)[0][:4]
    assert st.prefetch(cold, 0, rule) == 0
    assert st.n_miss[0] == 0
    for f in ("table", "map_cold", "slot_expert", "slot_stamp", "step"):
        assert np.array_equal(getattr(st, f), getattr(before, f)), f


def test_bad_arguments_rejected():
    st = State(8, 4)
    for E, S, mi, mk in ((0, 4, 4, 1), (8, 0, 4, 1), (8, 1025, 4, 1), (8, 4, -1, 1),
                         (8, 4, 1025, 1), (8, 4, 4, -1)):
        ids = np.zeros(1, np.int32)
        rc = oracle.lib().oracle_prefetch(
            oracle._ptr(ids), mk, E, S, mi, oracle._ptr(st.table), oracle._ptr(st.map_cold),
            oracle._ptr(st.slot_expert), oracle._ptr(st.slot_stamp), oracle._ptr(st.routed),
            oracle._ptr(st.miss), oracle._ptr(st.n_miss), 1)
        assert rc == -1, (E, S, mi, mk)


def _decays(before: State, ids, policy, decay) -> bool:
    """Would manage(ids) on `before` age the LFU counts (an inserting step on a multiple of
    decay)?"""
    if policy != LFU or decay <= 0 or (before.step[0] + 1) % decay:
        return False
    routed = np.unique(ids[(ids >= 0) & (ids < before.E)])
    return bool((before.table[routed] < 0).any())


@pytest.mark.parametrize("rule", ["rank", "serial"])
@pytest.mark.parametrize("policy,decay", [(LRU, 64), (LFU, 0), (LFU, 64), (LFU, 3)])
@pytest.mark.parametrize("workload,S", [("single-layer-e128", 16), ("single-layer-e128", 64),
                                        ("48-layer-e128-batch4", 48),
                                        ("8-layer-e256-fp8", 128)])
def test_right_prediction_is_invisible(workload, S, policy, decay, rule):
    from vllm_expert_cache import traces

    w = traces.WORKLOADS[workload]
    ids = traces.routing(w, 2, steps=400)
    E = w.experts
    base = State(E, S)
    checked = 0
    for t in range(ids.shape[0]):
        row = ids[t]
        md = min(E, row.size)
        a = base.copy()
        assert a.prefetch(row, S, rule) == 0
        pf_pairs = a.misses()
        assert base.manage(row, md, S, policy, decay, rule) == 0
        if _decays_after(base, policy, decay):
            continue  # the real step aged the counts; prefetch moved that step's inserts out
        assert a.manage(row, md, S, policy, decay, rule) == 0
        assert a.n_miss[0] == 0
        assert pf_pairs == base.misses(), t
        for f in POLICY_FIELDS:
            assert np.array_equal(getattr(a, f), getattr(base, f)), (t, f)
        checked += 1
    assert checked > ids.shape[0] // 2


def _decays_after(after: State, policy, decay) -> bool:
    """Did the manage step that produced `after` age the counts?"""
    return (policy == LFU and decay > 0 and after.step[0] % decay == 0
            and after.n_miss[0] > 0)


@pytest.mark.parametrize("policy", [LRU, LFU])
def test_decay_step_is_the_only_difference(policy):
    """On the LFU steps that age the counts, the states may differ; every other step they
    may not (the other test checks equality; this one checks the skip is exercised only
    where the rule says)."""
    from vllm_expert_cache import traces

    w = traces.WORKLOADS["single-layer-e128"]
    ids = traces.routing(w, 4, steps=300)
    base = State(128, 16)
    skipped = 0
    for t in range(ids.shape[0]):
        before = base.copy()
        assert base.manage(ids[t], 8, 16, policy, 8) == 0
        assert _decays(before, ids[t], policy, 8) == _decays_after(base, policy, 8)
        skipped += _decays_after(base, policy, 8)
    assert (skipped > 0) == (policy == LFU)


@pytest.mark.parametrize("seed", range(40))
def test_serial_equals_rank_on_random_predictions(seed):
    rng = np.random.default_rng(7000 + seed)
    E = int(rng.choice([1, 7, 64, 128, 257, 1000]))
    S = int(rng.choice([1, 3, 16, 64, 65, 129, 300]))
    mk = int(rng.choice([0, 1, 8, 33, 257]))
    mi = int(rng.choice([0, 1, 4, S]))
    nhot = int(rng.integers(0, min(S, E) + 1))
    hot, slots = rng.choice(E, nhot, replace=False), rng.choice(S, nhot, replace=False)
    a, b = State(E, S, miss_cap=max(mi, 1)), State(E, S, miss_cap=max(mi, 1))
    stamps = rng.integers(0, 1000, size=S)
    for st in (a, b):
        st.table[hot] = slots
        st.map_cold[hot] = -1
        st.slot_expert[slots] = hot
        st.slot_stamp[:] = stamps
    for t in range(8):
        ids = rng.integers(-3, E + 3, size=mk).astype(np.int32)
        routed = np.unique(ids[(ids >= 0) & (ids < E)])
        resident = {int(e): int(b.table[e]) for e in routed if b.table[e] >= 0}
        assert a.prefetch(ids, mi, "serial") == 0
        assert b.prefetch(ids, mi, "rank") == 0
        for f in State.FIELDS:
            assert np.array_equal(getattr(a, f), getattr(b, f)), (seed, t, f)
        _check_invariants(b)
        # a predicted expert is never evicted to make room for another
        assert all(b.table[e] == s for e, s in resident.items())
        assert all(b.table[e] >= 0 for e, _ in b.misses())


@pytest.mark.parametrize("policy", [LRU, LFU])
def test_wrong_predictions_keep_the_real_step_whole(policy):
    """Predictions that are half wrong: after each real step every routed expert is
    resident, the invariants hold, and an unused prefetched expert is the first victim."""
    from vllm_expert_cache import traces

    w = traces.WORKLOADS["single-layer-e128"]
    ids = traces.routing(w, 9, steps=400)
    rng = np.random.default_rng(9)
    st = State(128, 32)
    for t in range(ids.shape[0] - 1):
        nxt = ids[t + 1]
        pred = nxt.copy()
        wrong = rng.random(pred.size) < 0.5
        pred[wrong] = rng.integers(0, 128, wrong.sum())
        assert st.prefetch(pred, 8) == 0
        _check_invariants(st)
        fetched = [e for e, _ in st.misses()]
        assert all(st.slot_stamp[st.table[e]] == -1 for e in fetched)
        assert st.manage(nxt, 8, 32, policy, 64) == 0
        assert (st.table[np.unique(nxt)] >= 0).all()
        _check_invariants(st)
        assert (st.slot_stamp >= 0).all()  # every pending install was settled
        for e in fetched:
            if e not in set(nxt.tolist()):
                assert st.table[e] < 0 and st.map_cold[e] == e  # dropped


def _pending_state():
    """8 experts in 5 slots at step 9: experts 0 and 4 resident in slots 0 and 4 (stamps 3
    and 6); experts 2, 5 and 7 pending in slots 1, 2 and 3 (stamp -1)."""
    st = State(8, 5)
    st.slot_expert[:] = [0, 2, 5, 7, 4]
    st.slot_stamp[:] = [3, -1, -1, -1, 6]
    for s_, e in enumerate(st.slot_expert.tolist()):
        st.table[e], st.map_cold[e] = s_, -1
    st.step[0] = 9
    return st


@pytest.mark.parametrize("rule", ["rank", "serial"])
@pytest.mark.parametrize("policy", [LRU, LFU])
def test_hand_worked_settle_of_pending_installs(policy, rule):
    st = _pending_state()
    # routed {0, 5, 6}: 5 (slot 2) is confirmed, 2 (slot 1) and 7 (slot 3) are dropped; 0 is
    # a plain hit; 6 misses and takes the lowest key among the slots not routed: slots 1 and
    # 3 are now empty with stamp 0, so slot 1
    assert st.manage([6, 0, 5, 0], 4, 5, policy, 0, rule) == 0
    fresh = 10 if policy == LRU else 1
    hit0 = 10 if policy == LRU else 4
    assert st.misses() == [(6, 1)]
    assert st.slot_expert.tolist() == [0, 6, 5, -1, 4]
    assert st.slot_stamp.tolist() == [hit0, fresh, fresh, 0, 6]
    assert st.table.tolist() == [0, -1, -1, -1, 4, 2, 1, -1]
    assert st.map_cold.tolist() == [-1, 1, 2, 3, -1, -1, -1, 7]


@pytest.mark.parametrize("rule", ["rank", "serial"])
def test_confirmed_stamp_is_set_after_ageing(rule):
    """LFU step 10 with decay 5 inserts (expert 6 misses), so it ages: a confirmed pending
    slot ends at 1, as an install of this step does (ageing it, or counting it as a hit,
    would give 0)."""
    st = _pending_state()
    assert st.manage([6, 0, 5], 3, 5, LFU, 5, rule) == 0
    assert st.step[0] == 10
    assert st.slot_stamp.tolist() == [2, 1, 1, 0, 3]  # hit 3+1 and 6 halved, installs 1


@pytest.mark.parametrize("policy", [LRU, LFU])
def test_pending_installs_settle_once_and_survive_read_through(policy):
    st = _pending_state()
    # a wide step reads through: nothing is settled
    assert st.manage([0, 2, 5, 6], 3, 5, policy, 0) == 0
    assert st.slot_stamp.tolist() == [3, -1, -1, -1, 6] and st.step[0] == 10
    # served: 2 and 5 confirmed, 7 dropped
    assert st.manage([2, 5], 2, 5, policy, 0) == 0
    assert (st.slot_stamp >= 0).all() and st.table[7] < 0
    # the next step does not route 2 or 5: they stay resident (settled already)
    assert st.manage([0], 1, 5, policy, 0) == 0
    assert st.table[2] == 1 and st.table[5] == 2


def test_prefetch_evicts_pending_installs_first():
    st = _pending_state()
    # predicted {1, 3}: neither resident; the lowest keys among slots not predicted are the
    # pending ones (stamp -1), by slot: 1 then 2
    assert st.prefetch([3, 1], 4) == 0
    assert st.misses() == [(1, 1), (3, 2)]
    assert st.slot_expert.tolist() == [0, 1, 3, 7, 4]
    assert st.table[2] == -1 and st.table[5] == -1 and st.map_cold[5] == 5


@pytest.mark.parametrize("rule", ["rank", "serial"])
@pytest.mark.parametrize("policy,decay", [(LRU, 0), (LFU, 0), (LFU, 4)])
def test_wrong_prediction_leaves_only_its_evictions(policy, decay, rule):
    """prefetch(P) then manage(R) with P disjoint from R equals manage(R) on the state the
    prefetch left, with the predicted experts' slots emptied at stamp 0 (their previous
    experts stay evicted)."""
    from vllm_expert_cache import traces

    w = traces.WORKLOADS["single-layer-e128"]
    ids = traces.routing(w, 5, steps=300)
    rng = np.random.default_rng(11)
    st = State(128, 32)
    checked = 0
    for t in range(ids.shape[0]):
        row = ids[t]
        if t % 3 == 0:
            routed = set(row.tolist())
            cand = np.array([e for e in range(128) if e not in routed], np.int32)
            pred = rng.choice(cand, 4, replace=False)
            assert st.prefetch(pred, 4, rule) == 0
            emptied = st.copy()
            for e, s_ in st.misses():
                emptied.table[e], emptied.map_cold[e] = -1, e
                emptied.slot_expert[s_], emptied.slot_stamp[s_] = -1, 0
            assert emptied.manage(row, 8, 32, policy, decay, rule) == 0
            assert st.manage(row, 8, 32, policy, decay, rule) == 0
            for f in POLICY_FIELDS + ("miss", "n_miss"):
                assert np.array_equal(getattr(st, f), getattr(emptied, f)), (t, f)
            checked += 1
        else:
            assert st.manage(row, 8, 32, policy, decay, rule) == 0
        _check_invariants(st)
    assert checked == 100
