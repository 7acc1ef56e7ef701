"""Standalone remap and fused (manage + moe_align_block_size) parity on the GPU.

Remap is pinned by its closed form: torch advanced indexing `table[ids.long()]`, including
the wrap of negative ids (vllm_expert_cache/cache.py:108-110); ids outside [-E, E), where
torch raises, give -1. Fused is checked against the oracle on every step and against the
reference's own fused kernel (oracle/_ref) where that is deterministic (mk <= 256).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle
from test_oracle import align_lengths
from vllm_expert_cache import traces

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("n", [1, 8, 255, 4096, 100_000])
def test_remap_matches_torch_indexing(dtype, n):
    g = torch.Generator(device=gu.DEV).manual_seed(n)
    E = 256
    table = torch.randint(-1, 128, (E,), dtype=torch.int32, device=gu.DEV, generator=g)
    ids = torch.randint(-E, E, (n,), dtype=dtype, device=gu.DEV, generator=g)
    out = torch.empty_like(ids)
    nbytes = 8 if dtype == torch.int64 else 4
    assert gu.lib().expert_cache_remap(gu.ptr(ids), n, nbytes, gu.ptr(table), E, gu.ptr(out),
                                       gu.stream()) == 0
    want = table[ids.long()].to(dtype)
    assert torch.equal(out, want)


def test_remap_out_of_range_gives_minus_one():
    E = 16
    table = torch.arange(E, dtype=torch.int32, device=gu.DEV)
    ids = torch.tensor([16, -17, 1 << 30, -(1 << 30), 3, -1], dtype=torch.int32, device=gu.DEV)
    out = torch.empty_like(ids)
    assert gu.lib().expert_cache_remap(gu.ptr(ids), 6, 4, gu.ptr(table), E, gu.ptr(out),
                                       gu.stream()) == 0
    assert out.cpu().tolist() == [-1, -1, -1, -1, 3, 15]


def _fused_call(h, st: gu.Layers, ids_t, mk, bs, L, NB, outs):
    return h.expert_cache_fused(
        gu.ptr(ids_t), mk, st.E, st.S, min(st.E, mk), st.S, st.row("table", 0),
        st.row("map_cold", 0), st.row("slot_expert", 0), st.row("slot_stamp", 0),
        st.row("routed", 0), st.row("step", 0), st.row("miss", 0), st.row("n_miss", 0),
        bs, L, NB, *[gu.ptr(outs[k]) for k in ("sorted_hot", "eids_hot", "npad_hot",
                                               "sorted_cold", "eids_cold", "npad_cold")],
        gu.stream())


def _outs(L, NB):
    return {k: torch.full((n,), -5, dtype=torch.int32, device=gu.DEV) for k, n in
            (("sorted_hot", L), ("eids_hot", NB), ("npad_hot", 1),
             ("sorted_cold", L), ("eids_cold", NB), ("npad_cold", 1))}


@pytest.mark.parametrize("bs", [1, 16, 64])
@pytest.mark.parametrize("name,S", [("48-layer-e128", 16), ("48-layer-e128-batch4", 48),
                                    ("8-layer-e256-fp8", 128)])
def test_fused_matches_oracle_and_reference(name, S, bs):
    w = traces.WORKLOADS[name]
    ids = traces.routing(w, 2, 60)
    ids[::5, 1] = -1                      # padding ids are skipped on both sides
    E, mk = w.experts, ids.shape[1]
    L, NB = align_lengths(mk, E, bs)
    rh = gu.ref_lib()
    mine, theirs = gu.Layers(1, E, S), gu.Layers(1, E, S)
    ref = oracle.State(E, S)
    d_ids = torch.as_tensor(ids, device=gu.DEV)
    for t in range(ids.shape[0]):
        o_m, o_r = _outs(L, NB), _outs(L, NB)
        assert _fused_call(gu.lib(), mine, d_ids[t], mk, bs, L, NB, o_m) == 0
        rc, want = ref.fused(ids[t], min(E, mk), S, bs, L, NB)
        assert rc == 0
        if rh is not None:
            assert _fused_call(rh, theirs, d_ids[t], mk, bs, L, NB, o_r) == 0
        torch.cuda.synchronize()
        for k, v in want.items():
            assert np.array_equal(o_m[k].cpu().numpy(), v), (t, k)
            if rh is not None:
                assert torch.equal(o_r[k], o_m[k]), (t, k, "reference")
        assert np.array_equal(mine.table[0].cpu().numpy(), ref.table)
        assert np.array_equal(mine.slot_stamp[0].cpu().numpy(), ref.slot_stamp)
        assert np.array_equal(mine.miss[0].cpu().numpy(), ref.miss)


@pytest.mark.parametrize("mk", [1000, 13000])
def test_fused_wide_step_is_token_ordered(mk):
    """mk > 256 (a prefill-sized chunk): bucket contents in token order, and the same
    buckets as the reference's (which orders them by LDS atomics there). 13000 ids make
    outputs too large to build in LDS, so they take the path that fills memory first."""
    E, S, bs = 64, 32, 16
    rng = np.random.default_rng(4)
    ids = rng.integers(-2, E, size=mk).astype(np.int32)
    L, NB = align_lengths(ids.size, E, bs)
    st, ref = gu.Layers(1, E, S), oracle.State(E, S)
    outs = _outs(L, NB)
    d_ids = torch.as_tensor(ids, device=gu.DEV)
    assert _fused_call(gu.lib(), st, d_ids, ids.size, bs, L, NB, outs) == 0
    rc, want = ref.fused(ids, E, S, bs, L, NB)   # ~64 distinct misses, 32 slots: capped
    assert rc == 0
    torch.cuda.synchronize()
    for k, v in want.items():
        assert np.array_equal(outs[k].cpu().numpy(), v), k
    rh = gu.ref_lib()
    if rh is None:
        return
    theirs, o_r = gu.Layers(1, E, S), _outs(L, NB)
    assert _fused_call(rh, theirs, d_ids, ids.size, bs, L, NB, o_r) == 0
    torch.cuda.synchronize()
    for side in ("hot", "cold"):
        assert torch.equal(o_r[f"eids_{side}"], outs[f"eids_{side}"])
        assert torch.equal(o_r[f"npad_{side}"], outs[f"npad_{side}"])
        a = o_r[f"sorted_{side}"].cpu().numpy()
        b = outs[f"sorted_{side}"].cpu().numpy()
        e = outs[f"eids_{side}"].cpu().numpy()
        for bucket in np.unique(e[e >= 0]):  # same ids per bucket, in any order
            blocks = np.nonzero(e == bucket)[0]
            sl = slice(blocks[0] * bs, (blocks[-1] + 1) * bs)
            assert sorted(a[sl].tolist()) == sorted(b[sl].tolist()), (side, bucket)


@pytest.mark.parametrize("bs", [1, 3, 16])
@pytest.mark.parametrize("name,S", [("8-layer-e256-fp8", 128), ("48-layer-e128", 16)])
def test_fused_outputs_at_any_alignment(name, S, bs):
    """Output buffers 4 bytes past a 16-byte boundary take the scalar fill path; the bytes
    must be the same as with aligned buffers, and nothing outside the buffers changes, at
    128 and at 8 ids per step."""
    w = traces.WORKLOADS[name]
    ids = traces.routing(w, 1, 12)
    E, mk = w.experts, ids.shape[1]
    L, NB = align_lengths(mk, E, bs)
    ref = oracle.State(E, S)
    st = gu.Layers(1, E, S)
    d_ids = torch.as_tensor(ids, device=gu.DEV)
    for t in range(ids.shape[0]):
        backing = {k: torch.full((n + 2,), -7, dtype=torch.int32, device=gu.DEV) for k, n in
                   (("sorted_hot", L), ("eids_hot", NB), ("npad_hot", 1),
                    ("sorted_cold", L), ("eids_cold", NB), ("npad_cold", 1))}
        outs = {k: v[1:-1] for k, v in backing.items()}
        assert _fused_call(gu.lib(), st, d_ids[t], mk, bs, L, NB, outs) == 0
        rc, want = ref.fused(ids[t], min(E, mk), S, bs, L, NB)
        assert rc == 0
        torch.cuda.synchronize()
        for k, v in want.items():
            assert np.array_equal(outs[k].cpu().numpy(), v), (t, k)
            assert backing[k][0].item() == -7 and backing[k][-1].item() == -7, (t, k)


@pytest.mark.parametrize("mk", [0, 1, 7, 63, 64, 65, 200])
@pytest.mark.parametrize("bs", [1, 5, 16, 128])
def test_fused_random_ids_with_repeats(mk, bs):
    """Random ids with padding and repeats (several ids per bucket, buckets of several
    blocks), across one and several 64-id blocks of placement and block sizes that do and do
    not divide the counts, against the oracle on every output and the state, over four
    steps from a cold start."""
    E, S = 96, 24
    rng = np.random.default_rng(mk * 7 + bs)
    L, NB = align_lengths(max(mk, 1), E, bs)
    st, ref = gu.Layers(1, E, S), oracle.State(E, S)
    for t in range(4):
        ids = rng.integers(-3, E, size=mk).astype(np.int32)
        ids[rng.random(mk) < 0.3] = rng.integers(0, 6)        # a few popular experts
        outs = _outs(L, NB)
        d_ids = torch.as_tensor(ids, device=gu.DEV)
        assert _fused_call(gu.lib(), st, d_ids, mk, bs, L, NB, outs) == 0
        rc, want = ref.fused(ids, min(E, mk), S, bs, L, NB)
        assert rc == 0
        torch.cuda.synchronize()
        for k, v in want.items():
            assert np.array_equal(outs[k].cpu().numpy(), v), (t, k)
        assert np.array_equal(st.table[0].cpu().numpy(), ref.table), t
        assert np.array_equal(st.slot_stamp[0].cpu().numpy(), ref.slot_stamp), t


@pytest.mark.parametrize("mk", [8, 40, 130])
def test_fused_outputs_clipped_to_short_buffers(mk):
    """Buffers shorter than the padded totals (L and NB below the usual lengths): ids and
    block ids past the end are dropped, as the reference drops them."""
    E, S, bs = 64, 32, 4
    rng = np.random.default_rng(mk)
    L0, NB0 = align_lengths(mk, E, bs)
    st, ref = gu.Layers(1, E, S), oracle.State(E, S)
    for t, (L, NB) in enumerate(((L0 // 3, NB0 // 3), (5, 1), (L0, 2))):
        ids = rng.integers(0, E, size=mk).astype(np.int32)
        outs = _outs(L, NB)
        assert _fused_call(gu.lib(), st, torch.as_tensor(ids, device=gu.DEV), mk, bs, L, NB,
                           outs) == 0
        rc, want = ref.fused(ids, min(E, mk), S, bs, L, NB)
        assert rc == 0
        torch.cuda.synchronize()
        for k, v in want.items():
            assert np.array_equal(outs[k].cpu().numpy(), v), (t, k)
