"""Randomised policy-step parity: arbitrary shapes and arguments against the oracle.

Every case draws E (including above the 4096 experts held in LDS), S (including S > E and
S up to 1024), mk (including 0 and more than 256 ids), ids with padding and out-of-range
values, max_distinct (including below the routed count: read-through), max_inserts
(including 0 and caps below the miss count), policy and decay, and a random consistent warm
state with random stamps. Each step is compared on every field, and the fused remap output
against the closed form. The prefetch step runs over the same space, interleaved with
manage steps, and so does the one-launch pair of a policy step on one layer and a prefetch
step on another.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle

pytestmark = pytest.mark.gpu

CASES = 120
STEPS = 12


def _case(seed: int):
    rng = np.random.default_rng(seed)
    E = int(rng.choice([1, 2, 7, 64, 128, 200, 257, 512, 1000, 4096, 4100, 6000]))
    S = int(rng.choice([1, 2, 3, 16, 63, 64, 65, 128, 129, 300, 513, 1024]))
    mk = int(rng.choice([0, 1, 8, 33, 64, 200, 257, 300, 700]))
    mi = int(rng.choice([0, 1, 4, S, min(S + 5, 1024), 1024]))
    policy = int(rng.integers(0, 2))
    decay = int(rng.choice([0, 1, 3, 64]))
    nhot = int(rng.integers(0, min(S, E) + 1))
    hot = rng.choice(E, nhot, replace=False)
    slots = rng.choice(S, nhot, replace=False)
    stamps = rng.integers(0, 1000, size=S)
    return rng, E, S, mk, mi, policy, decay, hot, slots, stamps


def _device_state(E, S, mi, hot, slots, stamps):
    st = gu.Layers(1, E, S, miss_cap=max(mi, 1))
    table = np.full(E, -1, np.int32)
    cold = np.arange(E, dtype=np.int32)
    se = np.full(S, -1, np.int32)
    table[hot] = slots
    cold[hot] = -1
    se[slots] = hot
    st.table[0] = torch.as_tensor(table)
    st.map_cold[0] = torch.as_tensor(cold)
    st.slot_expert[0] = torch.as_tensor(se)
    st.slot_stamp[0] = torch.as_tensor(stamps)
    ref = oracle.State(E, S, miss_cap=max(mi, 1))
    ref.table[:], ref.map_cold[:], ref.slot_expert[:] = table, cold, se
    ref.slot_stamp[:] = stamps
    return st, ref


@pytest.mark.parametrize("seed", range(CASES))
def test_random_shapes(seed):
    rng, E, S, mk, mi, policy, decay, hot, slots, stamps = _case(seed)
    st, ref = _device_state(E, S, mi, hot, slots, stamps)
    fused_remap = seed % 2 == 0
    for t in range(STEPS):
        ids = rng.integers(-3, E + 3, size=mk).astype(np.int32)
        distinct = len(np.unique(ids[(ids >= 0) & (ids < E)]))
        md = int(rng.choice([distinct, distinct - 1, E, mk, -1]))
        d_ids = torch.as_tensor(ids, device=gu.DEV)
        out = torch.full((max(mk, 1),), -9, dtype=torch.int32, device=gu.DEV)
        rc = gu.manage_call(gu.lib(), st, 0, gu.ptr(d_ids) if mk else None, mk, md, mi,
                            policy, decay, gu.ptr(out) if fused_remap else None)
        assert rc == 0
        assert ref.manage(ids, md, mi, policy, decay) == 0
        torch.cuda.synchronize()
        tag = f"seed {seed} step {t}: E={E} S={S} mk={mk} md={md} mi={mi} pol={policy} dec={decay}"
        for name, dev in (("table", st.table[0]), ("map_cold", st.map_cold[0]),
                          ("slot_expert", st.slot_expert[0]), ("slot_stamp", st.slot_stamp[0]),
                          ("routed", st.routed[0]), ("step", st.step[0]), ("miss", st.miss[0]),
                          ("n_miss", st.n_miss[0])):
            got, want = dev.cpu().numpy(), getattr(ref, name)
            assert np.array_equal(got, want), f"{tag}: {name} differs at {gu.first_diff(got, want)}"
        if fused_remap and mk:
            assert np.array_equal(out.cpu().numpy()[:mk], oracle.remap(ids, ref.table)), tag


@pytest.mark.parametrize("seed", range(16))
def test_extreme_stamps(seed):
    """Warm states whose stamps spread over more than 2^31 (and whose keys overflow the
    20-bit shift, some negative), with enough misses per step for the many-insert search:
    its 64-bit form runs here, against the oracle's rank rule on every field."""
    rng = np.random.default_rng(1000 + seed)
    E = int(rng.choice([300, 1000, 4096]))
    S = int(rng.choice([65, 200, 257, 1024]))
    mk, mi = int(rng.choice([64, 200, 256])), S
    nhot = min(S, E) - int(rng.integers(0, 8))
    hot = rng.choice(E, nhot, replace=False)
    slots = rng.choice(S, nhot, replace=False)
    lo, hi = [(-(1 << 62), 1 << 62), (0, 1 << 45), (1 << 40, (1 << 40) + (1 << 33))][seed % 3]
    stamps = rng.integers(lo, hi, size=S)
    st, ref = _device_state(E, S, mi, hot, slots, stamps)
    policy, decay = seed % 2, int(rng.choice([0, 3]))
    for t in range(6):
        ids = rng.integers(0, E, size=mk).astype(np.int32)
        d_ids = torch.as_tensor(ids, device=gu.DEV)
        assert gu.manage_call(gu.lib(), st, 0, gu.ptr(d_ids), mk, mk, mi, policy, decay) == 0
        assert ref.manage(ids, mk, mi, policy, decay) == 0
        torch.cuda.synchronize()
        tag = f"seed {seed} step {t}: E={E} S={S} mk={mk} pol={policy} dec={decay} n_miss={ref.n_miss}"
        for name, dev in (("table", st.table[0]), ("map_cold", st.map_cold[0]),
                          ("slot_expert", st.slot_expert[0]), ("slot_stamp", st.slot_stamp[0]),
                          ("step", st.step[0]), ("miss", st.miss[0]), ("n_miss", st.n_miss[0])):
            got, want = dev.cpu().numpy(), getattr(ref, name)
            assert np.array_equal(got, want), f"{tag}: {name} differs at {gu.first_diff(got, want)}"


@pytest.mark.parametrize("seed", range(60))
def test_random_prefetch(seed):
    """The prefetch step over the same random shapes and warm states: each step runs a
    prefetch of random ids (padding and out-of-range included, any budget) into a miss
    list of its own, then a manage step, and both are compared on every field."""
    rng, E, S, mk, mi, policy, decay, hot, slots, stamps = _case(5000 + seed)
    pcap = max(S, 1024)
    st, ref = _device_state(E, S, mi, hot, slots, stamps)
    pf_miss = torch.zeros((2 * pcap,), dtype=torch.int32, device=gu.DEV)
    pf_n = torch.zeros((1,), dtype=torch.int32, device=gu.DEV)
    ref_pf, ref_pn = np.zeros(2 * pcap, np.int32), np.zeros(1, np.int32)
    ref_big = oracle.State(E, S, miss_cap=pcap)  # carries the prefetch's miss list
    for t in range(STEPS):
        pk = int(rng.choice([0, 1, 8, mk, 300]))
        budget = int(rng.choice([0, 1, 4, S, 1024]))
        pred = rng.integers(-3, E + 3, size=pk).astype(np.int32)
        d_pred = torch.as_tensor(pred, device=gu.DEV)
        rc = gu.lib().expert_cache_prefetch(
            gu.ptr(d_pred) if pk else None, pk, E, S, budget, st.row("table", 0),
            st.row("map_cold", 0), st.row("slot_expert", 0), st.row("slot_stamp", 0),
            st.row("routed", 0), gu.ptr(pf_miss), gu.ptr(pf_n), gu.stream())
        assert rc == 0
        for f in ("table", "map_cold", "slot_expert", "slot_stamp", "routed", "step"):
            setattr(ref_big, f, getattr(ref, f))  # shared arrays: one state, two miss lists
        ref_big.miss[:], ref_big.n_miss[:] = ref_pf, ref_pn
        assert ref_big.prefetch(pred, budget) == 0
        ref_pf, ref_pn = ref_big.miss.copy(), ref_big.n_miss.copy()
        torch.cuda.synchronize()
        tag = f"seed {seed} step {t}: E={E} S={S} pk={pk} budget={budget}"
        for name, dev, want in (("table", st.table[0], ref.table),
                                ("map_cold", st.map_cold[0], ref.map_cold),
                                ("slot_expert", st.slot_expert[0], ref.slot_expert),
                                ("slot_stamp", st.slot_stamp[0], ref.slot_stamp),
                                ("routed", st.routed[0], ref.routed), ("step", st.step[0], ref.step),
                                ("pf_miss", pf_miss, ref_pf), ("pf_n", pf_n, ref_pn)):
            got = dev.cpu().numpy()
            assert np.array_equal(got, want), f"{tag}: {name} differs at {gu.first_diff(got, want)}"
        ids = rng.integers(-3, E + 3, size=mk).astype(np.int32)
        d_ids = torch.as_tensor(ids, device=gu.DEV)
        md = min(E, mk)
        assert gu.manage_call(gu.lib(), st, 0, gu.ptr(d_ids) if mk else None, mk, md, mi,
                              policy, decay) == 0
        assert ref.manage(ids, md, mi, policy, decay) == 0
        torch.cuda.synchronize()
        for name, dev in (("table", st.table[0]), ("slot_expert", st.slot_expert[0]),
                          ("slot_stamp", st.slot_stamp[0]), ("step", st.step[0]),
                          ("miss", st.miss[0]), ("n_miss", st.n_miss[0])):
            got, want = dev.cpu().numpy(), getattr(ref, name)
            assert np.array_equal(got, want), f"{tag} (manage): {name} differs at {gu.first_diff(got, want)}"


@pytest.mark.parametrize("seed", range(40))
def test_random_one_launch(seed):
    """expert_cache_manage_remap_prefetch over the same random space: two layers with the
    same E and S and their own warm states; each step one layer's policy step and remap
    (int32 or int64 ids, any max_distinct) and the other layer's prefetch (any ids, any
    budget) run as one launch, and both layers are compared on every field."""
    rng, E, S, mk, mi, policy, decay, hot, slots, stamps = _case(9000 + seed)
    layers = [_device_state(E, S, mi, hot, slots, stamps)]
    nhot = int(rng.integers(0, min(S, E) + 1))
    layers.append(_device_state(E, S, mi, rng.choice(E, nhot, replace=False),
                                rng.choice(S, nhot, replace=False),
                                rng.integers(0, 1000, size=S)))
    pcap = 1024
    pf = [(torch.zeros((2 * pcap,), dtype=torch.int32, device=gu.DEV),
           torch.zeros((1,), dtype=torch.int32, device=gu.DEV)) for _ in range(2)]
    ref_pf = [(np.zeros(2 * pcap, np.int32), np.zeros(1, np.int32)) for _ in range(2)]
    side = oracle.State(E, S, miss_cap=pcap)  # carries a prefetch's miss list
    for t in range(STEPS):
        j = int(rng.integers(0, 2))
        k = 1 - j
        (st_j, ref_j), (st_k, ref_k) = layers[j], layers[k]
        ids = rng.integers(-3, E + 3, size=mk).astype(np.int32)
        distinct = len(np.unique(ids[(ids >= 0) & (ids < E)]))
        md = int(rng.choice([distinct, distinct - 1, E, mk]))
        idb = int(rng.choice([4, 8]))
        d_ids = torch.as_tensor(ids.astype(np.int64 if idb == 8 else np.int32), device=gu.DEV)
        out = torch.full((max(mk, 1),), -9, dtype=d_ids.dtype, device=gu.DEV)
        pk = int(rng.choice([0, 1, 8, mk, 300]))
        budget = int(rng.choice([0, 1, 4, S, 1024]))
        pred = rng.integers(-3, E + 3, size=pk).astype(np.int32)
        d_pred = torch.as_tensor(pred, device=gu.DEV)
        rc = gu.lib().expert_cache_manage_remap_prefetch(
            gu.ptr(d_ids) if mk else None, idb, mk, E, S, md, mi, st_j.row("table", 0),
            st_j.row("map_cold", 0), st_j.row("slot_expert", 0), st_j.row("slot_stamp", 0),
            st_j.row("routed", 0), st_j.row("step", 0), st_j.row("miss", 0),
            st_j.row("n_miss", 0), policy, decay, gu.ptr(out), gu.ptr(d_pred) if pk else None,
            pk, budget, st_k.row("table", 0), st_k.row("map_cold", 0),
            st_k.row("slot_expert", 0), st_k.row("slot_stamp", 0), st_k.row("routed", 0),
            gu.ptr(pf[k][0]), gu.ptr(pf[k][1]), gu.stream())
        assert rc == 0
        assert ref_j.manage(ids, md, mi, policy, decay) == 0
        for f in ("table", "map_cold", "slot_expert", "slot_stamp", "routed", "step"):
            setattr(side, f, getattr(ref_k, f))  # shared arrays: one state, two miss lists
        side.miss[:], side.n_miss[:] = ref_pf[k]
        assert side.prefetch(pred, budget) == 0
        ref_pf[k] = side.miss.copy(), side.n_miss.copy()
        torch.cuda.synchronize()
        tag = (f"seed {seed} step {t}: E={E} S={S} mk={mk} md={md} mi={mi} id{8 * idb} "
               f"pk={pk} budget={budget} manage on layer {j}")
        for l, (st, ref) in enumerate(layers):
            for name, dev in (("table", st.table[0]), ("map_cold", st.map_cold[0]),
                              ("slot_expert", st.slot_expert[0]),
                              ("slot_stamp", st.slot_stamp[0]), ("routed", st.routed[0]),
                              ("step", st.step[0]), ("miss", st.miss[0]),
                              ("n_miss", st.n_miss[0])):
                got, want = dev.cpu().numpy(), getattr(ref, name)
                assert np.array_equal(got, want), \
                    f"{tag}: layer {l} {name} differs at {gu.first_diff(got, want)}"
            for name, dev, want in (("pf_miss", pf[l][0], ref_pf[l][0]),
                                    ("pf_n", pf[l][1], ref_pf[l][1])):
                got = dev.cpu().numpy()
                assert np.array_equal(got, want), \
                    f"{tag}: layer {l} {name} differs at {gu.first_diff(got, want)}"
        if mk:
            assert np.array_equal(out.cpu().numpy()[:mk], oracle.remap(ids, ref_j.table)), tag
