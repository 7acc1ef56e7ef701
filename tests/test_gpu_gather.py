"""Gather parity on the GPU: after every step, each slot named in the miss list holds exactly
the bytes of its expert's rows from host memory, for every buffer -- and nothing else in the
slot buffers changes (kernels/expert_cache.hip:284-314 semantics).

Sources are pinned host memory read through its device address, as vLLM's expert offloader
provides it. Sizes cover tiles that do not divide the slab, 16-byte slabs, repeated buffers
(the caller's padding), several grid shapes, and the real expert layouts of the workloads.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle
from vllm_expert_cache import traces

pytestmark = pytest.mark.gpu

LFU = 1


class Expertstore:
    """E experts x buffers of random bytes in pinned host memory, plus S-slot HBM buffers."""

    def __init__(self, E: int, S: int, sizes, seed: int = 0):
        self.E, self.S, self.sizes = E, S, list(sizes)
        self.host = [gu.pinned(E * b) for b in self.sizes]
        for i, h in enumerate(self.host):
            gu.fill_random(h, seed * 100 + i)
        self.src = [gu.device_pointer(h) for h in self.host]
        self.dst = [torch.zeros(S * b, dtype=torch.uint8, device=gu.DEV) for b in self.sizes]

    def gather_args(self, order=None):
        order = list(range(len(self.sizes))) if order is None else order
        args = []
        for i in order:
            args += [gu.ptr(self.dst[i]), ctypes.c_void_p(self.src[i]),
                     ctypes.c_long(self.sizes[i])]
        return args

    def check_slot(self, sl: int, e: int) -> None:
        for i, b in enumerate(self.sizes):
            want = self.host[i][e * b:(e + 1) * b].to(gu.DEV, non_blocking=False)
            got = self.dst[i][sl * b:(sl + 1) * b]
            assert torch.equal(got, want), f"slot {sl} expert {e} buffer {i} ({b} B)"


def _drive(store: Expertstore, ids: np.ndarray, chunks: int, lanes: int, order=None,
           check_every: int = 1):
    """manage + gather per step on one layer; after each checked step every slot of the
    miss list must hold its expert's bytes, and slots outside it must be untouched."""
    E, S = store.E, store.S
    st = gu.Layers(1, E, S)
    ref = oracle.State(E, S)
    h = gu.lib()
    args = store.gather_args(order)
    while len(args) < 18:  # pad to six buffers with a repeat, as cache.refresh does
        args += args[-3:]
    d_ids = torch.as_tensor(ids, device=gu.DEV)
    for t in range(ids.shape[0]):
        before = [d.clone() for d in store.dst] if t % check_every == 0 else None
        rc = gu.manage_call(h, st, 0, gu.ptr(d_ids[t]), ids.shape[1], min(E, ids.shape[1]),
                            S, LFU, 64)
        assert rc == 0
        rc = h.expert_cache_gather(*args, st.row("miss", 0), st.row("n_miss", 0), chunks,
                                   lanes, gu.stream())
        assert rc == 0
        assert ref.manage(ids[t], min(E, ids.shape[1]), S, LFU, 64) == 0
        if before is None:
            continue
        torch.cuda.synchronize()
        pairs = ref.misses()
        assert int(st.n_miss[0, 0]) == len(pairs)
        for e, sl in pairs:
            store.check_slot(sl, e)
        touched = {sl for _, sl in pairs}
        for i, b in enumerate(store.sizes):
            for sl in range(S):
                if sl not in touched:
                    assert torch.equal(store.dst[i][sl * b:(sl + 1) * b],
                                       before[i][sl * b:(sl + 1) * b]), (t, sl, i)
    torch.cuda.synchronize()
    return st, ref


def _ids(E, k, T, seed):
    rng = np.random.default_rng(seed)
    return np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)


ODD_SIZES = [16, 48, 4096 + 16, 16 * 257, 1 << 16, 16 * 8191]


@pytest.mark.parametrize("chunks,lanes", [(1, 1), (3, 7), (16, 64), (32, 16), (64, 64)])
def test_gather_bit_identity_odd_sizes(chunks, lanes):
    store = Expertstore(40, 12, ODD_SIZES, seed=1)
    _drive(store, _ids(40, 6, 40, 2), chunks, lanes)


def test_gather_repeated_buffers_copied_once_and_correct():
    store = Expertstore(32, 8, [4096, 48, 16 * 1000], seed=3)
    # buffer 2 passed three times (as padding would), buffer 0 twice
    _drive(store, _ids(32, 4, 30, 4), 32, 16, order=[0, 1, 2, 2, 2, 0])


def test_gather_no_miss_writes_nothing():
    store = Expertstore(16, 8, [4096] * 6, seed=5)
    for d in store.dst:
        d.fill_(0xAB)
    n_miss = torch.zeros(1, dtype=torch.int32, device=gu.DEV)
    miss = torch.tensor([3, 1, 4, 2], dtype=torch.int32, device=gu.DEV)
    rc = gu.lib().expert_cache_gather(*store.gather_args(), gu.ptr(miss), gu.ptr(n_miss), 32,
                                      16, gu.stream())
    assert rc == 0
    torch.cuda.synchronize()
    assert all(bool((d == 0xAB).all()) for d in store.dst)


def test_gather_with_an_empty_miss_list_is_a_no_op():
    # a caller with max_inserts = 0 may pass a miss list with no capacity (a null pointer
    # here): the list is read only below n_miss, as kernels/expert_cache.hip:294-298 reads it
    store = Expertstore(16, 8, [4096] * 6, seed=6)
    for d in store.dst:
        d.fill_(0x5C)
    n_miss = torch.zeros(1, dtype=torch.int32, device=gu.DEV)
    miss = torch.empty(0, dtype=torch.int32, device=gu.DEV)
    slot_expert = torch.full((8,), -1, dtype=torch.int32, device=gu.DEV)
    h = gu.lib()
    rc = h.expert_cache_gather(*store.gather_args(), gu.ptr(miss), gu.ptr(n_miss), 32, 1,
                               gu.stream())
    assert rc == 0
    rc = h.expert_cache_gather_live(*store.gather_args(), gu.ptr(miss), gu.ptr(n_miss),
                                    gu.ptr(slot_expert), 16, 1, gu.stream())
    assert rc == 0
    torch.cuda.synchronize()
    assert all(bool((d == 0x5C).all()) for d in store.dst)


@pytest.mark.parametrize("name", ["48-layer-e128", "8-layer-e8-bf16"])
def test_gather_real_expert_layouts(name):
    """The workload's own expert layout and routing, one layer, default grid."""
    w = traces.WORKLOADS[name]
    steps = 120 if w.bytes_per_expert < (1 << 26) else 24
    store = Expertstore(w.experts, w.slots[-1] if len(w.slots) == 1 else 64,
                        [b.nbytes for b in w.buffers], seed=7)
    ids = traces.routing(w, 0, steps)
    st, ref = _drive(store, ids, 32, 16, check_every=4 if steps > 24 else 1)
    # every resident slot holds its expert's bytes at the end
    se = st.slot_expert[0].cpu().numpy()
    assert np.array_equal(se, ref.slot_expert)
    for sl, e in enumerate(se):
        if e >= 0:
            store.check_slot(sl, int(e))


def test_gather_matches_reference_kernel():
    """Same miss list through the reference's gather: identical slot bytes."""
    rh = gu.ref_lib()
    if rh is None:
        pytest.skip("reference library not built")
    sizes = [819200, 409600, 51200, 640, 25600, 2560]  # the reference's own test layout
    mine = Expertstore(64, 24, sizes, seed=11)
    theirs_dst = [torch.zeros_like(d) for d in mine.dst]
    ids = _ids(64, 10, 30, 12)
    st = gu.Layers(1, 64, 24)
    d_ids = torch.as_tensor(ids, device=gu.DEV)
    for t in range(ids.shape[0]):
        assert gu.manage_call(gu.lib(), st, 0, gu.ptr(d_ids[t]), 10, 10, 24, LFU, 64) == 0
        a_mine = mine.gather_args()
        a_ref = []
        for i, b in enumerate(sizes):
            a_ref += [gu.ptr(theirs_dst[i]), ctypes.c_void_p(mine.src[i]), ctypes.c_long(b)]
        tail = (st.row("miss", 0), st.row("n_miss", 0), 16, 64, gu.stream())
        assert gu.lib().expert_cache_gather(*a_mine, *tail) == 0
        assert rh.expert_cache_gather(*a_ref, *tail) == 0
    torch.cuda.synchronize()
    for a, b in zip(mine.dst, theirs_dst):
        assert torch.equal(a, b)


@pytest.mark.parametrize("chunks,lanes", [(32, 1), (16, 64)])
def test_gather_on_the_reference_suite_shape(chunks, lanes):
    """The reference's gather suite shape (tests/test_policy.py:234-282), our own seeds: 512
    experts, 257 slots, its six-buffer layout (1,308,800 B per expert), a warm start with
    257 experts in slot order, 40 steps of 5 tokens x 10 distinct ids, max_distinct 128,
    max_inserts 64, LRU. After every step each miss slab holds its expert's bytes; at the
    end every slot written during the run does too."""
    E, S, md, mi = 512, 257, 128, 64
    sizes = [819200, 409600, 51200, 640, 25600, 2560]
    store = Expertstore(E, S, sizes, seed=21)
    hot = sorted(np.random.default_rng(23).choice(E, S, replace=False).tolist())
    st = gu.Layers(1, E, S, miss_cap=mi, hot=hot)
    ref = oracle.State(E, S, hot=hot, miss_cap=mi)
    rng = np.random.default_rng(29)
    args = store.gather_args()
    written = {}
    for t in range(40):
        ids = np.concatenate([rng.choice(E, 10, replace=False) for _ in range(5)]).astype(np.int32)
        d_ids = torch.as_tensor(ids, device=gu.DEV)
        assert gu.manage_call(gu.lib(), st, 0, gu.ptr(d_ids), ids.size, md, mi, 0, 64) == 0
        assert gu.lib().expert_cache_gather(*args, st.row("miss", 0), st.row("n_miss", 0),
                                            chunks, lanes, gu.stream()) == 0
        assert ref.manage(ids, md, mi, 0, 64) == 0
        torch.cuda.synchronize()
        pairs = ref.misses()
        assert int(st.n_miss[0, 0]) == len(pairs)
        for e, sl in pairs:
            store.check_slot(sl, e)
            written[sl] = e
    assert len(written) > 64
    se = st.slot_expert[0].cpu().numpy()
    for sl, e in written.items():
        assert se[sl] == e
        store.check_slot(sl, e)


def _live_call(store: Expertstore, miss, n_miss, slot_expert, chunks=32, lanes=1):
    args = store.gather_args()
    while len(args) < 18:  # pad to six buffers with a repeat, as cache.refresh does
        args += args[-3:]
    return gu.lib().expert_cache_gather_live(*args, gu.ptr(miss), gu.ptr(n_miss),
                                             gu.ptr(slot_expert), chunks, lanes, gu.stream())


@pytest.mark.parametrize("chunks,lanes", [(1, 1), (3, 7), (32, 1), (64, 64)])
def test_gather_live_copies_live_pairs_like_gather(chunks, lanes):
    """expert_cache_gather_live with every pair live (slot_expert names each pair's expert):
    the same bytes as expert_cache_gather, and nothing outside the listed slots changes."""
    store = Expertstore(24, 10, ODD_SIZES, seed=7)
    for d in store.dst:
        d.fill_(0x5A)
    pairs = [(3, 0), (17, 4), (9, 7), (22, 9)]
    miss = torch.tensor([v for p in pairs for v in p], dtype=torch.int32, device=gu.DEV)
    n_miss = torch.tensor([len(pairs)], dtype=torch.int32, device=gu.DEV)
    slot_expert = torch.full((10,), -1, dtype=torch.int32, device=gu.DEV)
    for e, sl in pairs:
        slot_expert[sl] = e
    assert _live_call(store, miss, n_miss, slot_expert, chunks, lanes) == 0
    torch.cuda.synchronize()
    for e, sl in pairs:
        store.check_slot(sl, e)
    listed = {sl for _, sl in pairs}
    for i, b in enumerate(store.sizes):
        for sl in range(10):
            if sl not in listed:
                assert bool((store.dst[i][sl * b:(sl + 1) * b] == 0x5A).all())


def test_gather_live_stops_loading_dropped_pairs():
    """Pairs whose slot no longer names their expert (dropped, or given another expert)
    before the launch: each workgroup loads at most the first tile it meets of such a pair,
    so a 4.7 MB expert moves at most 32 workgroups x one 8 KB tile, and what lands is whole
    tiles of the right source bytes, the rest of the slot untouched. Live pairs in the same
    list are copied whole."""
    w = traces.WORKLOADS["48-layer-e128"]
    sizes = [b.nbytes for b in w.buffers]
    store = Expertstore(12, 6, sizes, seed=9)
    for d in store.dst:
        d.fill_(0x5A)
    pairs = [(2, 0), (5, 1), (7, 2), (11, 3)]
    miss = torch.tensor([v for p in pairs for v in p], dtype=torch.int32, device=gu.DEV)
    n_miss = torch.tensor([4], dtype=torch.int32, device=gu.DEV)
    slot_expert = torch.tensor([2, -1, 9, 11, -1, -1], dtype=torch.int32, device=gu.DEV)
    assert _live_call(store, miss, n_miss, slot_expert) == 0
    torch.cuda.synchronize()
    store.check_slot(0, 2)
    store.check_slot(3, 11)
    tile = 256 * 2 * 16
    for e, sl in ((5, 1), (7, 2)):
        copied = 0
        for i, b in enumerate(sizes):
            got = store.dst[i][sl * b:(sl + 1) * b]
            want = store.host[i][e * b:(e + 1) * b].to(gu.DEV)
            for t0 in range(0, b, tile):
                g, wv = got[t0:t0 + tile], want[t0:t0 + tile]
                if torch.equal(g, wv):
                    copied += 1
                else:
                    assert bool((g == 0x5A).all()), (e, i, t0)  # untouched, never partial
        assert copied <= 32, (e, copied)
