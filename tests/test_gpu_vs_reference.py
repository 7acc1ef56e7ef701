"""Head to head with the reference's own kernels on the same GPU.

The reference's kernels are compiled unchanged from kernels/expert_cache.hip into
oracle/_ref (these tests skip when that library is absent). Every comparison first checks
that both produce the same bytes, then compares their times on the same stream, both
captured in HIP graphs so that host launch cost is out of the picture:

  * the reference's timing shapes (tests/test_policy.py:283-318): E=512, S=257, 50 routing
    ids per step, LRU, six buffers of 1,308,800 B per expert; manage at steady state and
    gather of 1, 2, 8, 52 and 64 experts;
  * a decode loop (LFU, cold start) through each side's per-layer refresh: the reference's
    as cache.py:112-163 does it (manage, gather on its 16 x 64 default grid, torch remap),
    this library's as vllm_expert_cache/cache.py does it (manage with the fused remap,
    gather on its default grid). Four workloads: 48-layer-e128 (8 of its layers, 64 slots),
    its batch-4 form (48 slots), 352 MB bf16 experts (4 slots) and 44 MB fp8 experts
    (4 layers, 128 slots, 128 ids per step).

Each test prints one "speed:" line per figure (run pytest with -s to see them). The byte
checks come first. Then a regression guard: this library not slower than the reference
beyond a 10 % noise margin. By default it guards the comparisons where this library leads
clearly (the policy step at the reference's timing shape, the decode loops of the 4.7 MB
and 352 MB experts, the fused kernel); where both sides run at the host link's rate (the
gathers of the reference's shapes, the batch-4 and 44 MB decode loops) the times are
reported only. EC_SPEED_ASSERT=1 guards every comparison, EC_SPEED_ASSERT=0 none (for a
run under a profiler, whose per-dispatch cost swamps kernels of a few microseconds).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest
import torch

import gpu_util as gu
from vllm_expert_cache import traces
from vllm_expert_cache.cache import DEFAULT_CHUNKS, DEFAULT_LANES

pytestmark = pytest.mark.gpu

LRU, LFU = 0, 1
REF_CHUNKS, REF_LANES = 16, 64      # vllm_expert_cache/cache.py:96-97 of the reference
REF_SIZES = (819200, 409600, 51200, 640, 25600, 2560)   # tests/test_policy.py:237


SPEED_ASSERT = os.environ.get("EC_SPEED_ASSERT")  # "1": every comparison, "0": none
# a regression guard, not the measurement (the timings are printed); ties at the link's rate
# get room for noise
MARGIN = 1.10


def _not_slower(this: float, reference: float, clear_lead: bool = True) -> bool:
    """Times (lower is better): this within MARGIN of the reference, where guarded."""
    guarded = SPEED_ASSERT == "1" or (SPEED_ASSERT != "0" and clear_lead)
    return not guarded or this <= reference * MARGIN


def _ref():
    h = gu.ref_lib()
    if h is None:
        pytest.skip("reference library not built (oracle/_ref)")
    return h


def _graph_us(launch, reps: int) -> float:
    """Mean µs per launch of `reps` launches captured in one graph, replayed 3 times."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            launch()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(3):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / (3 * reps)


def _timed_loop(g, ids_static, ids_dev, T: int) -> float:
    """ms for T decode steps: each step copies its routing ids into the graph's input and
    replays the graph (the graph's state is reset by the caller beforehand). Every step is
    queued behind a stream hold before the first event."""
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    # hold the stream while the steps are queued, so that a loop whose steps are shorter
    # than the host's launch time is not timed at the host's launch rate
    torch.cuda._sleep(int(5e7))
    a.record()
    for t in range(T):
        ids_static.copy_(ids_dev[t], non_blocking=True)
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b)


def _say(*a):
    print("speed:", *a, flush=True)


# ---- the reference's own timing shapes ----------------------------------------------------

def _drive_512(h):
    """tests/test_policy.py:244-252 shape: warm start with 257 of 512 experts resident, then
    40 steps of 5 tokens x 10 distinct ids, max_distinct 128, max_inserts 64, LRU."""
    E, S = 512, 257
    hot = sorted(np.random.default_rng(3).choice(E, S, replace=False).tolist())
    st = gu.Layers(1, E, S, miss_cap=64, hot=hot)
    rng = np.random.default_rng(11)
    for _ in range(40):
        ids = np.stack([rng.choice(E, size=10, replace=False) for _ in range(5)]).ravel()
        d = torch.as_tensor(ids.astype(np.int32), device=gu.DEV)
        assert gu.manage_call(h, st, 0, gu.ptr(d), 50, 128, 64, LRU, 64) == 0
    torch.cuda.synchronize()
    return st


def test_manage_steady_state_vs_reference():
    """tests/test_policy.py:312-321: 50 routing ids, repeated, on the driven state."""
    ref = _ref()
    mine, theirs = _drive_512(gu.lib()), _drive_512(ref)
    for f in ("table", "map_cold", "slot_expert", "slot_stamp", "step", "n_miss"):
        assert torch.equal(getattr(mine, f), getattr(theirs, f)), f
    ids = np.stack([np.random.default_rng(k).choice(512, 10, replace=False)
                    for k in range(5)]).ravel()
    d = torch.as_tensor(ids.astype(np.int32), device=gu.DEV)
    us = {}
    for name, h, st in (("reference", ref, theirs), ("this", gu.lib(), mine)):
        us[name] = _graph_us(lambda: gu.manage_call(h, st, 0, gu.ptr(d), 50, 128, 64, LRU, 64),
                             200)
    for f in ("table", "map_cold", "slot_expert", "slot_stamp", "step", "n_miss"):
        assert torch.equal(getattr(mine, f), getattr(theirs, f)), f
    _say(f"manage E=512 S=257 mk=50 steady state: reference {us['reference']:.2f} us, "
         f"this {us['this']:.2f} us ({us['reference'] / us['this']:.1f}x)")
    assert _not_slower(us["this"], us["reference"])


@pytest.fixture(scope="module")
def store_512():
    E, S = 512, 257
    host = [gu.pinned(E * b) for b in REF_SIZES]
    for i, t in enumerate(host):
        gu.fill_random(t, 70 + i)
    src = [gu.device_pointer(t) for t in host]
    return E, S, host, src


@pytest.mark.parametrize("n", [1, 2, 8, 52, 64])
def test_gather_vs_reference(store_512, n):
    """tests/test_policy.py:285-310: n experts per launch, miss list (j, j)."""
    ref = _ref()
    _, S, host, src = store_512
    miss = torch.arange(n, dtype=torch.int32, device=gu.DEV).repeat_interleave(2)
    n_miss = torch.tensor([n], dtype=torch.int32, device=gu.DEV)
    per_expert = sum(REF_SIZES)
    us = {}
    for name, h, grid in (("reference", ref, (REF_CHUNKS, REF_LANES)),
                          ("this", gu.lib(), (DEFAULT_CHUNKS, DEFAULT_LANES))):
        dst = [torch.zeros(S * b, dtype=torch.uint8, device=gu.DEV) for b in REF_SIZES]
        args = []
        for i, b in enumerate(REF_SIZES):
            args += [gu.ptr(dst[i]), ctypes.c_void_p(src[i]), ctypes.c_long(b)]
        tail = (gu.ptr(miss), gu.ptr(n_miss), grid[0], grid[1])

        def launch():
            assert h.expert_cache_gather(*args, *tail, gu.stream()) == 0

        us[name] = _graph_us(launch, 20)
        for i, b in enumerate(REF_SIZES):
            want = host[i][:n * b].to(gu.DEV)
            assert torch.equal(dst[i][:n * b], want), (name, i)
            assert not dst[i][n * b:].any(), (name, i)
    gbs = {k: n * per_expert / (v * 1e-6) / 1e9 for k, v in us.items()}
    _say(f"gather {n:2d} x {per_expert} B: reference {us['reference']:.1f} us "
         f"({gbs['reference']:.1f} GB/s), this {us['this']:.1f} us ({gbs['this']:.1f} GB/s)")
    assert _not_slower(us["this"], us["reference"], clear_lead=False)


# ---- the 48-layer-e128 decode loop through each side's refresh -----------------------------

@pytest.mark.parametrize("name,S,L,T", [("48-layer-e128", 64, 8, 512),
                                         ("48-layer-e128-batch4", 48, 8, 512),
                                         ("8-layer-e8-bf16", 4, 8, 96),
                                         ("8-layer-e256-fp8", 128, 4, 48)])
def test_decode_loop_vs_reference(name, S, L, T):
    ref = _ref()
    w = traces.WORKLOADS[name]
    E, mk = w.experts, w.mk
    bufs = [b.nbytes for b in w.buffers]
    B_exp = sum(bufs)
    ids_np = np.stack([traces.routing(w, l, T) for l in range(L)], axis=1)
    ids_dev = torch.as_tensor(ids_np, device=gu.DEV)
    host = [gu.pinned(E * b) for b in bufs]     # one store read by every layer
    for i, t in enumerate(host):
        gu.fill_random(t, 90 + i)
    src = [gu.device_pointer(t) for t in host]
    P = ctypes.c_void_p

    def row(t, l):
        return P(t.data_ptr() + l * t.stride(0) * t.element_size())

    runs = {}
    workload = name
    for name in ("reference", "this"):
        h = ref if name == "reference" else gu.lib()
        st = gu.Layers(L, E, S)
        slots = [[torch.zeros(S * b, dtype=torch.uint8, device=gu.DEV) for b in bufs]
                 for _ in range(L)]
        ids_static = torch.zeros((L, mk), dtype=torch.int32, device=gu.DEV)
        out_static = torch.zeros((L, mk), dtype=torch.int32, device=gu.DEV)
        out_hist = torch.zeros((T, L, mk), dtype=torch.int32, device=gu.DEV)
        nm_hist = torch.zeros((T, L), dtype=torch.int32, device=gu.DEV)
        g_args = []
        for l in range(L):
            a = []
            for i in range(6):  # padded to six with a repeat, as both refresh paths do
                j = min(i, len(bufs) - 1)
                a += [gu.ptr(slots[l][j]), P(src[j]), ctypes.c_long(bufs[j])]
            g_args.append(a)
        grid = (REF_CHUNKS, REF_LANES) if name == "reference" else (DEFAULT_CHUNKS,
                                                                      DEFAULT_LANES)

        def launch(h=h, st=st, g_args=g_args, grid=grid, ids_static=ids_static,
                   out_static=out_static, name=name):
            s = gu.stream()
            for l in range(L):
                common = (st.row("table", l), st.row("map_cold", l), st.row("slot_expert", l),
                          st.row("slot_stamp", l), st.row("routed", l), st.row("step", l),
                          st.row("miss", l), st.row("n_miss", l), LFU, 64)
                if name == "reference":
                    rc = h.expert_cache_manage(row(ids_static, l), mk, E, S, min(E, mk), S,
                                               *common, s)
                else:
                    rc = h.expert_cache_manage_remap(row(ids_static, l), 4, mk, E, S,
                                                     min(E, mk), S, *common,
                                                     row(out_static, l), s)
                assert rc == 0
                rc = h.expert_cache_gather(*g_args[l], st.row("miss", l), st.row("n_miss", l),
                                           grid[0], grid[1], s)
                assert rc == 0
                if name == "reference":  # cache.py:108-110 of the reference
                    out_static[l].copy_(
                        st.table[l][ids_static[l].to(torch.int64)].to(torch.int32))

        fields = ("table", "map_cold", "slot_expert", "slot_stamp", "routed", "step", "miss",
                  "n_miss")
        snap = [getattr(st, f).clone() for f in fields]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            launch()  # warm-up outside capture, then the state is reset to a cold start
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        for f, v in zip(fields, snap):
            getattr(st, f).copy_(v)
        for per_layer in slots:
            for t in per_layer:
                t.zero_()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            launch()
        torch.cuda.synchronize()
        for t in range(T):  # parity pass, recording every step
            ids_static.copy_(ids_dev[t], non_blocking=True)
            g.replay()
            out_hist[t].copy_(out_static, non_blocking=True)
            nm_hist[t].copy_(st.n_miss[:, 0], non_blocking=True)
        torch.cuda.synchronize()
        final = [getattr(st, f).clone() for f in fields]
        runs[name] = dict(final=final, slots=[[t.clone() for t in p] for p in slots],
                          out=out_hist, nm=nm_hist)
        for f, v in zip(fields, snap):
            getattr(st, f).copy_(v)
        runs[name]["ms"] = _timed_loop(g, ids_static, ids_dev, T)
        del slots, st
        torch.cuda.empty_cache()

    r, m = runs["reference"], runs["this"]
    assert torch.equal(r["nm"], m["nm"])
    assert torch.equal(r["out"], m["out"])
    for f, x, y in zip(fields, r["final"], m["final"]):
        assert torch.equal(x, y), f
    for l in range(L):
        for i in range(len(bufs)):
            assert torch.equal(r["slots"][l][i], m["slots"][l][i]), (l, i)
    inserts = int(m["nm"].sum())
    assert inserts > 0
    gb = inserts * B_exp / 1e9
    _say(f"decode loop {workload} ({L} layers x {T} steps, S={S}, LFU, {inserts} inserts, "
         f"{gb:.1f} GB): reference {r['ms']:.1f} ms ({gb / r['ms'] * 1e3:.1f} GB/s), "
         f"this {m['ms']:.1f} ms ({gb / m['ms'] * 1e3:.1f} GB/s)")
    assert _not_slower(m["ms"], r["ms"],
                       clear_lead=name in ("48-layer-e128", "8-layer-e8-bf16"))


# ---- expert_cache_fused: the LRU step plus both moe_align_block_size outputs ---------------

@pytest.mark.parametrize("name,S", [("48-layer-e128", 64), ("48-layer-e128-batch4", 48),
                                    ("8-layer-e256-fp8", 128)])
def test_fused_vs_reference(name, S):
    """Each side's fused kernel over a decode loop (8 layers x 256 steps, block size 16): same
    outputs and state on every step (mk <= 256, where the reference is token-ordered)."""
    from test_oracle import align_lengths

    ref = _ref()
    w = traces.WORKLOADS[name]
    Lyr, T, E, mk, bs = 8, 256, w.experts, w.mk, 16
    Lw, NB = align_lengths(mk, E, bs)
    ids_dev = torch.as_tensor(np.stack([traces.routing(w, l, T) for l in range(Lyr)], axis=1),
                              device=gu.DEV)
    keys = ("sorted_hot", "eids_hot", "npad_hot", "sorted_cold", "eids_cold", "npad_cold")
    sizes = dict(sorted_hot=Lw, eids_hot=NB, npad_hot=1, sorted_cold=Lw, eids_cold=NB,
                 npad_cold=1)
    runs = {}
    for side, h in (("reference", ref), ("this", gu.lib())):
        st = gu.Layers(Lyr, E, S)
        ids_static = torch.zeros((Lyr, mk), dtype=torch.int32, device=gu.DEV)
        outs = {k: torch.zeros((Lyr, n), dtype=torch.int32, device=gu.DEV)
                for k, n in sizes.items()}
        hist = {k: torch.zeros((T, Lyr, n), dtype=torch.int32, device=gu.DEV)
                for k, n in sizes.items()}

        def launch(h=h, st=st, ids_static=ids_static, outs=outs):
            for l in range(Lyr):
                rc = h.expert_cache_fused(
                    ctypes.c_void_p(ids_static.data_ptr() + l * mk * 4), mk, E, S,
                    min(E, mk), S, st.row("table", l), st.row("map_cold", l),
                    st.row("slot_expert", l), st.row("slot_stamp", l), st.row("routed", l),
                    st.row("step", l), st.row("miss", l), st.row("n_miss", l), bs, Lw, NB,
                    *[ctypes.c_void_p(outs[k].data_ptr() + l * sizes[k] * 4) for k in keys],
                    gu.stream())
                assert rc == 0

        fields = ("table", "map_cold", "slot_expert", "slot_stamp", "routed", "step", "miss",
                  "n_miss")
        snap = [getattr(st, f).clone() for f in fields]
        side_stream = torch.cuda.Stream()
        side_stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side_stream):
            launch()
        torch.cuda.current_stream().wait_stream(side_stream)
        torch.cuda.synchronize()
        for f, v in zip(fields, snap):
            getattr(st, f).copy_(v)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            launch()
        torch.cuda.synchronize()
        for t in range(T):  # parity pass, recording every step
            ids_static.copy_(ids_dev[t], non_blocking=True)
            g.replay()
            for k in keys:
                hist[k][t].copy_(outs[k], non_blocking=True)
        torch.cuda.synchronize()
        final = [getattr(st, f).clone() for f in fields]
        for f, v in zip(fields, snap):
            getattr(st, f).copy_(v)
        runs[side] = dict(ms=_timed_loop(g, ids_static, ids_dev, T), final=final, hist=hist)

    r, m = runs["reference"], runs["this"]
    for k in keys:
        assert torch.equal(r["hist"][k], m["hist"][k]), k
    for f, x, y in zip(fields, r["final"], m["final"]):
        assert torch.equal(x, y), f
    per = {s: v["ms"] * 1e3 / (T * Lyr) for s, v in runs.items()}
    _say(f"fused {name} (E={E} S={S} mk={mk} bs={bs}, {Lyr} layers x {T} steps): reference "
         f"{per['reference']:.2f} us/layer-step, this {per['this']:.2f} us/layer-step "
         f"({per['reference'] / per['this']:.1f}x)")
    assert _not_slower(per["this"], per["reference"])
