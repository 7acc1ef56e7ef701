"""The plugin path end to end on the GPU, at layer level: arming (backends/generic.py), the
wrapped `apply`, `ExpertSlotCache.refresh` (policy step + fused remap + gather) and the
slot-bound expert computation, inside a small MoE decode loop.

The reference claims greedy outputs byte-identical with and without the cache
(README.md:216-247) but has no test for it. Here two identical 4-layer MoE stacks run the
same decode. One is armed with the cache (8 of 32 experts resident per layer); the other
reads the full expert tensors. Every step's output must be bit-identical. The expert math
is plain fp32 torch, the same operations on the same values, whether it reads slots with
slot ids or the full tensors with expert ids. Steps wider than the slot budget take the
read-through path. The armed decode step is also captured in a HIP graph and replayed.
"""
from __future__ import annotations

import types

import numpy as np
import pytest
import torch

import gpu_util as gu
from test_generic import new_log, quant_config
from vllm_expert_cache.backends import generic

pytestmark = pytest.mark.gpu

E, S, H, I, K, LAYERS = 32, 8, 64, 32, 2, 4


class MoELayer(torch.nn.Module):
    """Expert tensors registered as Parameters on the GPU, like vLLM's FusedMoE layer. The
    router's gate lives outside the layer, as in vLLM."""

    def __init__(self, seed: int):
        super().__init__()
        g = torch.Generator(device=gu.DEV).manual_seed(seed)
        self.w13_weight = torch.nn.Parameter(
            torch.randn(E, 2 * I, H, device=gu.DEV, generator=g) * 0.05, requires_grad=False)
        self.w2_weight = torch.nn.Parameter(
            torch.randn(E, H, I, device=gu.DEV, generator=g) * 0.05, requires_grad=False)
        self.global_num_experts = E
        self.expert_map = None


class TorchMoE:
    """A FusedMoEMethodBase stand-in whose apply computes the MoE in fp32 torch from
    whatever expert tensors and ids it is given."""

    is_monolithic = False

    def __init__(self, layer):
        self.moe_quant_config = self.get_fused_moe_quant_config(layer)
        self.moe_kernel = types.SimpleNamespace(
            fused_experts=types.SimpleNamespace(quant_config=self.moe_quant_config))

    def get_fused_moe_quant_config(self, layer):
        return quant_config()

    def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None,
              shared_experts_input=None):
        ids = topk_ids.reshape(-1).long()
        w13 = layer.w13_weight[ids].contiguous()               # [T*K, 2I, H]
        w2 = layer.w2_weight[ids].contiguous()                 # [T*K, H, I]
        xr = x.repeat_interleave(K, dim=0).unsqueeze(-1)       # [T*K, H, 1]
        h = torch.bmm(w13, xr).squeeze(-1)                     # [T*K, 2I]
        act = torch.nn.functional.silu(h[:, :I]) * h[:, I:]
        y = torch.bmm(w2, act.unsqueeze(-1).contiguous()).squeeze(-1)  # [T*K, H]
        return (y.view(-1, K, H) * topk_weights.unsqueeze(-1)).sum(1)


def _route(gate, x):
    w, ids = torch.topk(torch.softmax(x @ gate.t(), dim=-1), K, dim=-1)
    return w, ids.to(torch.int32)


def _forward(layers, methods, gates, x):
    for layer, m, gate in zip(layers, methods, gates):
        w, ids = _route(gate, x)
        x = x + m.apply(layer, x, w, ids)
    return x


def _model(armed: bool):
    layers = [MoELayer(100 + l) for l in range(LAYERS)]
    methods = [TorchMoE(layer) for layer in layers]
    gates = [torch.randn(E, H, device=gu.DEV,
                         generator=torch.Generator(device=gu.DEV).manual_seed(200 + l))
             for l in range(LAYERS)]
    if armed:
        for layer, m in zip(layers, methods):
            assert generic.arm(layer, m, new_log("e2e").logger)
    return layers, methods, gates


@pytest.mark.parametrize("policy", ["lfu", "lru"])
def test_decode_outputs_identical_with_the_cache(monkeypatch, policy):
    monkeypatch.setenv("EXPERT_CACHE_SLOTS", str(S))
    monkeypatch.setenv("EXPERT_CACHE_POLICY", policy)
    cached = _model(True)
    full = _model(False)
    caches = [layer._expert_cache for layer in cached[0]]
    rng = np.random.default_rng(17)
    g = torch.Generator(device=gu.DEV).manual_seed(3)
    read_through = 0
    for t in range(64):
        tokens = 5 if t % 16 == 15 else int(rng.integers(1, 5))   # 5 x 2 ids > 8 slots
        x = torch.randn(tokens, H, device=gu.DEV, generator=g)
        steps_before = [int(c.step[0]) for c in caches]
        a = _forward(*cached, x)
        b = _forward(*full, x)
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"step {t}: max |diff| {float((a - b).abs().max())}"
        steps_after = [int(c.step[0]) for c in caches]
        if tokens * K > S:
            read_through += 1
            assert steps_after == steps_before  # read-through: the policy did not run
        else:
            assert all(s1 == s0 + 1 for s0, s1 in zip(steps_before, steps_after))
    assert read_through == 4
    for c in caches:
        assert int(c.step[0]) == 60
        resident = c.slot_expert[c.slot_expert >= 0].long()
        for n in ("w13_weight", "w2_weight"):
            src = getattr(c.owner, n).data
            assert torch.equal(c.slots[n][c.slot_expert >= 0], src[resident]), n


def test_decode_step_graph_captured(monkeypatch):
    monkeypatch.setenv("EXPERT_CACHE_SLOTS", str(S))
    cached = _model(True)
    full = _model(False)
    static_x = torch.zeros(2, H, device=gu.DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _forward(*cached, static_x)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = _forward(*cached, static_x)
    g = torch.Generator(device=gu.DEV).manual_seed(5)
    for t in range(32):
        static_x.copy_(torch.randn(2, H, device=gu.DEV, generator=g))
        graph.replay()
        want = _forward(*full, static_x.clone())
        torch.cuda.synchronize()
        assert torch.equal(static_out, want), f"replay {t}"
    assert all(int(layer._expert_cache.step[0]) == 33 for layer in cached[0])


def _forward_prefetching(layers, methods, gates, x, stats, along=False):
    """As _forward, and before each layer's MoE, the next layer's cache is prefetched with
    that layer's gate applied to the current hidden state (a pre-gated predictor). With
    `along`, the prefetch step is staged to run inside this layer's policy launch."""
    for l, (layer, m, gate) in enumerate(zip(layers, methods, gates)):
        if l + 1 < len(layers):
            _, pred = _route(gates[l + 1], x)
            nxt = layers[l + 1]._expert_cache
            if nxt.prefetch(pred, along=layer._expert_cache if along else None):
                stats["pred"].append(pred)
        w, ids = _route(gate, x)
        if l > 0:
            stats["real"].append(ids)
        x = x + m.apply(layer, x, w, ids)
    return x


@pytest.mark.parametrize("along", [False, True], ids=["own-launch", "along"])
def test_decode_with_next_layer_prefetch_identical(monkeypatch, along):
    monkeypatch.setenv("EXPERT_CACHE_SLOTS", str(S))
    cached = _model(True)
    full = _model(False)
    g = torch.Generator(device=gu.DEV).manual_seed(11)
    stats = {"pred": [], "real": []}
    fetched = 0
    for t in range(48):
        x = torch.randn(2, H, device=gu.DEV, generator=g)
        a = _forward_prefetching(*cached, x, stats, along)
        b = _forward(*full, x)
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"step {t}"
        fetched += sum(int(layer._expert_cache.pf_n_miss[0]) for layer in cached[0][1:])
    for layer in cached[0]:
        layer._expert_cache.join()
    hits = sum(len(set(p.flatten().tolist()) & set(r.flatten().tolist()))
               for p, r in zip(stats["pred"], stats["real"]))
    total = sum(len(set(r.flatten().tolist())) for r in stats["real"])
    print(f"pre-gated prediction: {hits}/{total} routed experts predicted; "
          f"{fetched} experts prefetched", flush=True)
    assert fetched > 0 and hits > 0


def test_decode_with_prefetch_along_graph_captured(monkeypatch):
    """The pre-gated decode step with every prefetch staged along the layer before, captured
    in one graph: each layer's policy launch carries the next layer's prefetch step."""
    monkeypatch.setenv("EXPERT_CACHE_SLOTS", str(S))
    cached = _model(True)
    full = _model(False)
    static_x = torch.zeros(2, H, device=gu.DEV)
    stats = {"pred": [], "real": []}
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _forward_prefetching(*cached, static_x, stats, along=True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = _forward_prefetching(*cached, static_x, stats, along=True)
    caches = [layer._expert_cache for layer in cached[0]]
    assert all(c._rider is None and c._riding_on is None and not c._pf_pending
               for c in caches)
    g = torch.Generator(device=gu.DEV).manual_seed(7)
    for t in range(32):
        static_x.copy_(torch.randn(2, H, device=gu.DEV, generator=g))
        graph.replay()
        want = _forward(*full, static_x.clone())
        torch.cuda.synchronize()
        assert torch.equal(static_out, want), f"replay {t}"
    assert all(int(c.step[0]) == 33 for c in caches)
    for c, layer in zip(caches, cached[0]):
        resident = c.slot_expert[c.slot_expert >= 0].long()
        for n in ("w13_weight", "w2_weight"):
            assert torch.equal(c.slots[n][c.slot_expert >= 0],
                               getattr(layer, n).data[resident]), n
