"""ExpertSlotCache end to end on the GPU: the plugin's host side driving the HIP path.

Sources are pinned host tensors read through unified addressing, as vLLM's offloader
leaves them. Each refresh must return the oracle's slot ids, and every routed id's slot
must hold that expert's bytes afterwards. The refresh sequence must also survive HIP-graph
capture: replays with new routing match an eager twin cache step for step.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import gpu_util as gu
import oracle
from vllm_expert_cache.cache import ExpertSlotCache

pytestmark = pytest.mark.gpu

E, S, K = 128, 32, 8


class Owner(torch.nn.Module):
    """Expert tensors in pinned host memory: int8 weights and fp32 scales."""

    def __init__(self, seed=0):
        super().__init__()
        g = torch.Generator().manual_seed(seed)

        def host(shape, dtype):
            t = torch.empty(shape, dtype=dtype, pin_memory=True)
            if dtype == torch.int8:
                t.copy_(torch.randint(-128, 128, shape, dtype=torch.int8, generator=g))
            else:
                t.copy_(torch.randn(shape, generator=g))
            return t

        self.w13_weight = host((E, 96, 64), torch.int8)
        self.w2_weight = host((E, 64, 48), torch.int8)
        self.w13_weight_scale = host((E, 96, 1), torch.float32)
        self.w2_weight_scale = host((E, 64, 1), torch.float32)


NAMES = ["w13_weight", "w2_weight", "w13_weight_scale", "w2_weight_scale"]


def _check_slots(cache: ExpertSlotCache, owner: Owner, ids: torch.Tensor, slot_ids):
    for e, sl in zip(ids.flatten().tolist(), slot_ids.flatten().tolist()):
        assert 0 <= sl < S
        for n in NAMES:
            want = getattr(owner, n)[e].to(gu.DEV)
            assert torch.equal(cache.slots[n][sl], want), (e, sl, n)


def test_unified_addressing_premise():
    t = gu.pinned(4096)
    assert gu.device_pointer(t) == t.data_ptr()


@pytest.mark.parametrize("policy", ["lfu", "lru"])
@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_refresh_matches_oracle(monkeypatch, policy, dtype):
    monkeypatch.setenv("EXPERT_CACHE_POLICY", policy)
    owner = Owner()
    cache = ExpertSlotCache(owner, NAMES, E, S, gu.DEV)
    ref = oracle.State(E, S)
    rng = np.random.default_rng(3)
    pol = 1 if policy == "lfu" else 0
    for t in range(80):
        tokens = 1 + t % 4
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(tokens)])
        d_ids = torch.as_tensor(ids, dtype=dtype, device=gu.DEV)
        assert cache.fits(d_ids)
        slot_ids = cache.refresh(d_ids)
        assert slot_ids.dtype == dtype and slot_ids.shape == d_ids.shape
        assert ref.manage(ids.ravel(), min(E, ids.size), S, pol, 64) == 0
        torch.cuda.synchronize()
        assert np.array_equal(slot_ids.cpu().numpy().ravel(), oracle.remap(
            ids.ravel().astype(np.int64), ref.table).astype(np.int64))
        assert np.array_equal(cache.table.cpu().numpy(), ref.table)
        assert np.array_equal(cache.slot_stamp.cpu().numpy(), ref.slot_stamp)
        _check_slots(cache, owner, d_ids, slot_ids)
        assert torch.equal(cache.remap(d_ids), slot_ids)
    wide = torch.zeros((5, K), dtype=dtype, device=gu.DEV)
    assert not cache.fits(wide)


def test_refresh_under_graph_capture():
    owner = Owner(1)
    eager = ExpertSlotCache(owner, NAMES, E, S, gu.DEV)
    graphed = ExpertSlotCache(owner, NAMES, E, S, gu.DEV)
    for c in (eager, graphed):
        for buf in c.slots.values():
            buf.zero_()
    rng = np.random.default_rng(8)
    static_ids = torch.zeros((2, K), dtype=torch.int32, device=gu.DEV)

    # warm up on a side stream, as torch requires before capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        graphed.refresh(static_ids)
        eager.refresh(static_ids)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out = graphed.refresh(static_ids)

    for t in range(40):
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(2)]).astype(np.int32)
        static_ids.copy_(torch.as_tensor(ids, device=gu.DEV))
        g.replay()
        want = eager.refresh(static_ids.clone())
        torch.cuda.synchronize()
        assert torch.equal(static_out, want), t
        for f in ("table", "map_cold", "slot_expert", "slot_stamp", "step", "miss", "n_miss"):
            assert torch.equal(getattr(graphed, f), getattr(eager, f)), (t, f)
        for n in NAMES:
            assert torch.equal(graphed.slots[n], eager.slots[n]), (t, n)
        _check_slots(graphed, owner, static_ids, static_out)


def test_refresh_follows_a_source_that_moves():
    """vLLM's offloader may rebind an expert tensor after the cache was built. The next
    refresh must gather from where the tensor is now: new misses hold the new source's
    bytes. A source moved to host memory the GPU cannot read is refused."""
    owner = Owner(7)
    cache = ExpertSlotCache(owner, NAMES, E, S, gu.DEV)
    first = torch.arange(0, K, dtype=torch.int32, device=gu.DEV)
    cache.refresh(first)
    torch.cuda.synchronize()
    _check_slots(cache, owner, first, cache.remap(first))
    key = cache._gather_key
    moved = torch.empty_like(owner.w13_weight, pin_memory=True)
    moved.copy_(torch.randint(-128, 128, tuple(moved.shape), dtype=torch.int8))
    owner.w13_weight = moved
    second = torch.arange(K, 2 * K, dtype=torch.int32, device=gu.DEV)
    slot_ids = cache.refresh(second)
    torch.cuda.synchronize()
    assert cache._gather_key != key
    _check_slots(cache, owner, second, slot_ids)
    owner.w13_weight = moved.clone()  # pageable
    before = {f: getattr(cache, f).clone() for f in ("table", "slot_expert", "slot_stamp", "step")}
    with pytest.raises(ValueError, match="pin it"):
        cache.refresh(torch.arange(2 * K, 3 * K, dtype=torch.int32, device=gu.DEV))
    torch.cuda.synchronize()
    for f, t in before.items():  # refused before the policy step ran
        assert torch.equal(getattr(cache, f), t), f


class WideOwner(torch.nn.Module):
    """Eight per-expert tensors in pinned host memory (weights, scales, zero points and
    biases of odd widths), more than one gather call's six buffers."""

    SHAPES = {"w13_weight": ((E, 96, 64), torch.int8), "w2_weight": ((E, 64, 48), torch.int8),
              "w13_weight_scale": ((E, 96, 1), torch.float32),
              "w2_weight_scale": ((E, 64, 1), torch.float32),
              "w13_weight_zero": ((E, 96, 4), torch.int8), "w2_weight_zero": ((E, 64, 4), torch.int8),
              "w13_bias": ((E, 96), torch.float32), "w2_bias": ((E, 64), torch.bfloat16)}

    def __init__(self, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        for n, (shape, dtype) in self.SHAPES.items():
            t = torch.empty(shape, dtype=dtype, pin_memory=True)
            t.view(torch.uint8).copy_(torch.randint(0, 256, t.view(torch.uint8).shape,
                                                    dtype=torch.uint8, generator=g))
            setattr(self, n, t)


def test_refresh_with_more_tensors_than_one_gather_takes():
    """Eight mirrored tensors take two gather calls per refresh (six buffers each, the second
    padded with repeats). After every step, eagerly and with a prefetch along the refresh,
    every resident slot of every tensor holds its expert's bytes."""
    names = list(WideOwner.SHAPES)
    owners = [WideOwner(1), WideOwner(2)]
    caches = [ExpertSlotCache(o, names, E, S, gu.DEV) for o in owners]
    assert all(len(c.names) == 8 for c in caches)
    rng = np.random.default_rng(8)
    for t in range(30):
        ids = [torch.as_tensor(np.stack([rng.choice(E, K, replace=False) for _ in range(2)])
                               .astype(np.int32), device=gu.DEV) for _ in range(2)]
        pred = torch.as_tensor(rng.choice(E, K, replace=False).astype(np.int32), device=gu.DEV)
        if t % 2:
            caches[1].prefetch(pred, along=caches[0])
        caches[0].refresh(ids[0])
        caches[1].refresh(ids[1])
        torch.cuda.synchronize()
        for c, o in zip(caches, owners):
            live = torch.nonzero(c.slot_expert >= 0).flatten()
            experts = c.slot_expert[live].long().cpu()
            for n in names:  # bytes: random bits read as floats include NaNs
                want = getattr(o, n)[experts].view(torch.uint8)
                assert torch.equal(c.slots[n][live].cpu().view(torch.uint8), want), (t, n)
