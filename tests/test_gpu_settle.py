"""Pending prefetch installs settled by every entry point that runs a real policy step.

A prefetch step installs its predictions as pending (stamp -1); the next served step of
expert_cache_manage, expert_cache_manage_remap (int32 and int64 ids),
expert_cache_manage_remap_prefetch (its policy workgroup) or expert_cache_fused confirms the
routed ones and drops the rest. Each case builds pending installs with a real
expert_cache_prefetch call, then runs a fixed sequence through one entry point: a wide step
that reads through (pending installs must survive it), a served step on an LFU ageing step
with other misses (a confirmed install must end at stamp 1), and a few more steps. Every
field of the state, the miss list and the slot ids must equal the oracle's after each call.
Shapes cover one slot per lane, eight slots per lane with the table beyond the registers,
and experts beyond the LDS table.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle

pytestmark = pytest.mark.gpu

LRU, LFU = 0, 1
SHAPES = [(64, 16, 8), (600, 300, 40), (5000, 100, 24)]  # E, S, ids per step
ENTRIES = ["manage", "manage_remap_i32", "manage_remap_i64", "manage_remap_prefetch", "fused"]


def _align_lengths(mk, E, bs):
    L = min(mk * bs, mk + E * (bs - 1)) if mk < E else mk + E * (bs - 1)
    return L, -(-L // bs)


def _words(s: oracle.State) -> np.ndarray:
    return np.concatenate([s.table, s.map_cold, s.slot_expert, s.slot_stamp.view(np.int32),
                           s.step.view(np.int32)])


# expert_cache_fused takes at most 1024 experts, so it runs on the first two shapes only
CASES = [(entry, *shape) for shape in SHAPES for entry in ENTRIES
         if not (entry == "fused" and shape[0] > 1024)]


@pytest.mark.parametrize("entry,E,S,mk", CASES, ids=lambda v: str(v))
def test_pending_installs_settle_like_the_oracle(entry, E, S, mk):
    rng = np.random.default_rng(E * 31 + S)
    policy = LRU if entry == "fused" else LFU
    decay = 0 if entry == "fused" else 4
    h = gu.lib()
    st = gu.Layers(2, E, S)            # row 0: the layer under test; row 1: a prefetch partner
    ref = oracle.State(E, S)
    # warm state: every slot holds an expert, stamps 1..9, step 6 (the next served step is
    # step 7; step 8 is an ageing step under decay 4)
    hot = rng.choice(E, S, replace=False).astype(np.int32)
    stamps = rng.integers(1, 10, S)
    st.table[0, torch.as_tensor(hot, dtype=torch.int64, device=gu.DEV)] = \
        torch.arange(S, dtype=torch.int32, device=gu.DEV)
    st.map_cold[0, torch.as_tensor(hot, dtype=torch.int64, device=gu.DEV)] = -1
    st.slot_expert[0] = torch.as_tensor(hot, device=gu.DEV)
    st.slot_stamp[0] = torch.as_tensor(stamps, device=gu.DEV)
    st.step[0] = 6
    ref.table[hot] = np.arange(S, dtype=np.int32)
    ref.map_cold[hot] = -1
    ref.slot_expert[:] = hot
    ref.slot_stamp[:] = stamps
    ref.step[0] = 6

    cold = np.setdiff1d(np.arange(E), hot)
    pred = rng.choice(cold, min(mk, 6), replace=False).astype(np.int32)
    d_pred = torch.as_tensor(pred, device=gu.DEV)
    pf_miss = torch.zeros(2 * S, dtype=torch.int32, device=gu.DEV)
    pf_n = torch.zeros(1, dtype=torch.int32, device=gu.DEV)
    rc = h.expert_cache_prefetch(gu.ptr(d_pred), pred.size, E, S, S, st.row("table", 0),
                                 st.row("map_cold", 0), st.row("slot_expert", 0),
                                 st.row("slot_stamp", 0), st.row("routed", 0), gu.ptr(pf_miss),
                                 gu.ptr(pf_n), gu.stream())
    assert rc == 0
    keep_miss, keep_n = ref.miss.copy(), ref.n_miss.copy()
    assert ref.prefetch(pred, S) == 0
    ref.miss[:], ref.n_miss[:] = keep_miss, keep_n
    torch.cuda.synchronize()
    assert (ref.slot_stamp == -1).sum() == pred.size
    assert np.array_equal(st.state_words()[0].cpu().numpy(), _words(ref))

    # the steps: half the predictions routed (confirmed), half not (dropped)
    right = pred[: pred.size // 2]
    routed_hot = rng.choice(hot, mk, replace=False)
    wide = np.concatenate([routed_hot[: mk - right.size], right]).astype(np.int32)
    steps = [("read-through", wide, 1)]   # max_distinct 1 < distinct routed ids
    for t in range(5):
        new = rng.choice(np.setdiff1d(cold, pred), 2, replace=False)
        row = np.concatenate([right if t == 0 else rng.choice(hot, 2, replace=False), new,
                              rng.choice(hot, mk, replace=False)])[:mk].astype(np.int32)
        steps.append((f"served {t}", row, min(E, mk)))

    L, NB = _align_lengths(mk, E, 16)
    outs = {k: torch.zeros(n, dtype=torch.int32, device=gu.DEV) for k, n in
            (("sorted_hot", L), ("eids_hot", NB), ("npad_hot", 1), ("sorted_cold", L),
             ("eids_cold", NB), ("npad_cold", 1))}
    partner_pred = torch.as_tensor(rng.choice(E, 4, replace=False).astype(np.int32),
                                   device=gu.DEV)
    for tag, row, md in steps:
        if entry == "manage_remap_i64":
            d_ids = torch.as_tensor(row.astype(np.int64), device=gu.DEV)
        else:
            d_ids = torch.as_tensor(row, device=gu.DEV)
        out = torch.full_like(d_ids, -9)
        common = (st.row("table", 0), st.row("map_cold", 0), st.row("slot_expert", 0),
                  st.row("slot_stamp", 0), st.row("routed", 0), st.row("step", 0),
                  st.row("miss", 0), st.row("n_miss", 0))
        if entry == "manage":
            rc = h.expert_cache_manage(gu.ptr(d_ids), mk, E, S, md, S, *common, policy, decay,
                                       gu.stream())
        elif entry.startswith("manage_remap_i"):
            rc = h.expert_cache_manage_remap(gu.ptr(d_ids), d_ids.element_size(), mk, E, S, md,
                                             S, *common, policy, decay, gu.ptr(out),
                                             gu.stream())
        elif entry == "manage_remap_prefetch":
            pf = (st.row("table", 1), st.row("map_cold", 1), st.row("slot_expert", 1),
                  st.row("slot_stamp", 1), st.row("routed", 1), st.row("miss", 1),
                  st.row("n_miss", 1))
            rc = h.expert_cache_manage_remap_prefetch(
                gu.ptr(d_ids), 4, mk, E, S, md, S, *common, policy, decay, gu.ptr(out),
                gu.ptr(partner_pred), 4, S, *pf, gu.stream())
        else:
            rc = h.expert_cache_fused(gu.ptr(d_ids), mk, E, S, md, S, *common, 16, L, NB,
                                      *[gu.ptr(outs[k]) for k in outs], gu.stream())
        assert rc == 0, (tag, rc)
        if entry == "fused":
            rc_ref, want_out = ref.fused(row, md, S, 16, L, NB)
            assert rc_ref == 0
        else:
            assert ref.manage(row, md, S, policy, decay) == 0
        torch.cuda.synchronize()
        assert np.array_equal(st.state_words()[0].cpu().numpy(), _words(ref)), tag
        assert int(st.n_miss[0, 0]) == int(ref.n_miss[0]), tag
        assert np.array_equal(st.miss[0].cpu().numpy(), ref.miss), tag
        if entry.startswith("manage_remap") and md >= len(set(row.tolist())):
            assert np.array_equal(out.cpu().numpy(), oracle.remap(row.astype(
                out.cpu().numpy().dtype), ref.table)), tag
        if entry == "fused":
            for k, v in want_out.items():
                assert np.array_equal(outs[k].cpu().numpy(), v), (tag, k)
        if tag == "read-through":
            assert (ref.slot_stamp == -1).sum() == pred.size  # still pending
        elif tag == "served 0":
            assert (ref.slot_stamp >= 0).all()                # all settled
            for e in right:
                assert ref.table[e] >= 0
            for e in pred[pred.size // 2:]:
                assert ref.table[e] < 0 or e in row
