"""Arming logic of backends/generic.py on CPU, against stand-ins for vLLM's MoE classes.

The same fourteen situations the reference checks (tests/test_generic.py:142-352): which
tensors are mirrored, that a cached step sees slot storage and a slot-sized config, that a
wide step reads through, that the keyword call works, that the layer is restored, and that
every unsafe layout is refused with a reason. `refresh` is replaced by an identity so only
the binding is under test here; the kernels are covered by the GPU tests.
"""
from __future__ import annotations

from dataclasses import dataclass

import pytest
import torch

from vllm_expert_cache.backends import generic

E, S = 16, 4
H, N = 8, 12


@pytest.fixture(autouse=True)
def _slots(monkeypatch):
    monkeypatch.setenv("EXPERT_CACHE_SLOTS", str(S))
    torch.manual_seed(0)


class Log:
    def __init__(self):
        self.msgs = []

    def _rec(self, fmt, *a):
        self.msgs.append(fmt % a if a else fmt)

    warning = info = debug = _rec

    def said(self, needle):
        return any(needle in m for m in self.msgs)


@dataclass
class Desc:
    scale: torch.Tensor | None = None
    alpha_or_gscale: torch.Tensor | None = None
    zp: torch.Tensor | None = None
    bias: torch.Tensor | None = None


@dataclass
class Cfg:
    _a1: Desc
    _a2: Desc
    _w1: Desc
    _w2: Desc


class Experts:
    def __init__(self, cfg):
        self.quant_config = cfg


class Kernel:
    def __init__(self, cfg):
        self.fused_experts = Experts(cfg)


def _param(t):
    return torch.nn.Parameter(t, requires_grad=False)


class Layer(torch.nn.Module):
    """Expert tensors registered as Parameters, like vLLM's FusedMoE layer."""

    def __init__(self, extra=(), n_experts=E):
        super().__init__()
        self.w13_weight = _param(torch.randn(n_experts, N, H))
        self.w2_weight = _param(torch.randn(n_experts, H, N // 2))
        for name, shape in extra:
            setattr(self, name, _param(torch.randn(*shape)))
        self.global_num_experts = n_experts
        self.expert_map = None


class Method:
    """A FusedMoEMethodBase stand-in whose config factory reads `reads` off the layer."""

    is_monolithic = False

    def __init__(self, layer, reads=(), hidden=None):
        self.reads = list(reads)
        self.hidden = hidden
        self.moe_quant_config = self._cfg(layer)
        self.moe_kernel = Kernel(self.moe_quant_config)
        self.seen = None

    def _cfg(self, layer):
        got = [getattr(layer, n) for n in self.reads]
        w1 = Desc(scale=got[0] if len(got) > 0 else None, zp=got[2] if len(got) > 2 else None)
        w2 = Desc(scale=got[1] if len(got) > 1 else None, zp=got[3] if len(got) > 3 else None)
        if self.hidden is not None:
            w1.bias = self.hidden
        return Cfg(Desc(), Desc(), w1, w2)

    def get_fused_moe_quant_config(self, layer):
        return self._cfg(layer)

    def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None,
              shared_experts_input=None):
        self.seen = dict(w13=layer.w13_weight, w2=layer.w2_weight,
                         cfg=self.moe_kernel.fused_experts.quant_config, ids=topk_ids.clone(),
                         gne=layer.global_num_experts)
        return torch.zeros(1)


def arm(layer, method):
    log = Log()
    return generic.arm(layer, method, log), log


SCALES = [("w13_weight_scale", (E, N, 1)), ("w2_weight_scale", (E, H, 1))]
SCALE_NAMES = ["w13_weight_scale", "w2_weight_scale"]


def _stub_refresh(layer):
    layer._expert_cache.refresh = lambda ids: ids.clone()


def test_unquantized_mirrors_the_two_weights():
    layer = Layer()
    ok, _ = arm(layer, Method(layer))
    assert ok
    assert set(layer._expert_cache.names) == {"w13_weight", "w2_weight"}


def test_int8_mirrors_weights_and_scales():
    layer = Layer(SCALES)
    ok, _ = arm(layer, Method(layer, reads=SCALE_NAMES))
    assert ok
    assert set(layer._expert_cache.names) == {"w13_weight", "w2_weight", *SCALE_NAMES}


def test_wna16_mirrors_six_tensors():
    extra = SCALES + [("w13_weight_zero_point", (E, N, 1)), ("w2_weight_zero_point", (E, H, 1))]
    layer = Layer(extra)
    ok, _ = arm(layer, Method(layer, reads=[n for n, _ in extra]))
    assert ok
    assert len(layer._expert_cache.names) == 6


def test_packed_weights_with_alias_share_one_slot():
    layer = Layer()
    for base in ("w13", "w2"):
        t = getattr(layer, f"{base}_weight")
        del layer._parameters[f"{base}_weight"]
        layer.register_parameter(f"{base}_weight_packed", t)
        setattr(layer, f"{base}_weight", t)
    m = Method(layer)
    ok, log = arm(layer, m)
    assert ok, log.msgs
    cache = layer._expert_cache
    assert len(cache.slots) == 2
    assert set(cache.bound) == {"w13_weight", "w13_weight_packed", "w2_weight",
                                "w2_weight_packed"}
    assert cache.bound["w13_weight"].data_ptr() == cache.bound["w13_weight_packed"].data_ptr()
    _stub_refresh(layer)
    m.apply(layer, torch.randn(1, H), torch.ones(1, 2), torch.zeros(1, 2, dtype=torch.int32))
    assert m.seen["w13"].data_ptr() == cache.slots["w13_weight_packed"].data_ptr()
    assert layer.w13_weight.data_ptr() == layer.w13_weight_packed.data_ptr()


def test_wide_step_reads_through():
    layer = Layer(SCALES)
    m = Method(layer, reads=SCALE_NAMES)
    assert arm(layer, m)[0]
    wide = torch.zeros(1, S + 1, dtype=torch.int32)
    m.apply(layer, torch.randn(1, H), torch.ones(1, S + 1), wide)
    assert m.seen["cfg"]._w1.scale.size(0) == E
    assert m.seen["gne"] == E
    assert m.seen["w13"].data_ptr() == layer.w13_weight.data_ptr()


def test_fitting_step_is_bound_to_slots():
    layer = Layer(SCALES)
    m = Method(layer, reads=SCALE_NAMES)
    assert arm(layer, m)[0]
    cache = layer._expert_cache
    _stub_refresh(layer)
    m.apply(layer, torch.randn(1, H), torch.ones(1, 2), torch.zeros(1, 2, dtype=torch.int32))
    assert m.seen["w13"].data_ptr() == cache.slots["w13_weight"].data_ptr()
    assert m.seen["cfg"]._w1.scale.size(0) == S
    assert m.seen["gne"] == S


def test_apply_accepts_keyword_call():
    layer = Layer()
    m = Method(layer)
    assert arm(layer, m)[0]
    _stub_refresh(layer)
    m.apply(layer=layer, x=torch.randn(1, H), topk_weights=torch.ones(1, 2),
            topk_ids=torch.zeros(1, 2, dtype=torch.int32), shared_experts=None,
            shared_experts_input=None)
    assert m.seen is not None


def test_layer_is_restored():
    layer = Layer(SCALES)
    m = Method(layer, reads=SCALE_NAMES)
    names = ("w13_weight", "w2_weight", *SCALE_NAMES)
    before = {n: getattr(layer, n).data_ptr() for n in names}
    assert arm(layer, m)[0]
    _stub_refresh(layer)
    m.apply(layer, torch.randn(1, H), torch.ones(1, 2), torch.zeros(1, 2, dtype=torch.int32))
    assert {n: getattr(layer, n).data_ptr() for n in names} == before
    assert layer.global_num_experts == E
    assert m.moe_kernel.fused_experts.quant_config._w1.scale.size(0) == E


def test_hidden_per_expert_tensor_is_refused():
    layer = Layer()
    ok, log = arm(layer, Method(layer, hidden=torch.randn(E, N)))
    assert not ok
    assert log.said("stayed bound to full") and log.said("_w1.bias")


def test_monolithic_is_refused():
    layer = Layer()
    m = Method(layer)
    m.is_monolithic = True
    ok, log = arm(layer, m)
    assert not ok and log.said("monolithic")


def test_expert_parallel_is_refused():
    layer = Layer()
    layer.expert_map = torch.arange(E)
    ok, log = arm(layer, Method(layer))
    assert not ok and log.said("expert parallelism")


def test_ragged_auxiliary_is_caught_by_the_leak_check():
    layer = Layer([("w13_weight_scale", (E, 3))])  # 12 bytes per expert
    ok, log = arm(layer, Method(layer, reads=["w13_weight_scale"]))
    assert not ok
    assert log.said("stayed bound to full") and log.said("w13_weight_scale")


def test_ragged_weight_is_refused():
    layer = Layer()
    layer.w13_weight = _param(torch.randn(E, 3))
    ok, log = arm(layer, Method(layer))
    assert not ok
    assert log.said("multiple of 16") and log.said("w13_weight")


def test_nothing_to_cache(monkeypatch):
    monkeypatch.setenv("EXPERT_CACHE_SLOTS", str(E))
    layer = Layer()
    ok, _ = arm(layer, Method(layer))
    assert not ok


def test_no_recognised_weight_pair_is_reported():
    layer = Layer()
    t = layer.w13_weight
    del layer._parameters["w13_weight"]
    layer.register_parameter("w13_qweight", t)
    ok, log = arm(layer, Method.__new__(Method))
    assert not ok and log.said("no recognised expert weight pair")


def test_install_without_vllm_stays_out_of_the_way():
    log = Log()
    assert generic.install(log) is False
    assert log.said("vLLM MoE interfaces unavailable")


def test_prefetch_refuses_a_prediction_wider_than_the_slots():
    """Host-side prefetch rules that need no kernel: a prediction with more ids than slots
    is refused before anything is launched, and join() with nothing pending does nothing."""
    layer = Layer(SCALES)
    m = Method(layer, reads=SCALE_NAMES)
    assert arm(layer, m)[0]
    cache = layer._expert_cache
    assert cache.prefetch(torch.zeros(S + 1, dtype=torch.int32)) is False
    assert cache.prefetch(torch.zeros(1, S + 1, dtype=torch.int64)) is False
    cache.join()
    assert cache._pf_pending is False


def test_prefetch_along_stages_without_launching(monkeypatch):
    """Staging a prefetch along another layer's cache is host bookkeeping only: nothing is
    launched until that layer's refresh (or a join). Partners that cannot share one launch
    are refused: the same cache, or one with other expert or slot counts."""
    from vllm_expert_cache import cache as cache_mod

    def no_launch():
        raise AssertionError("staging must not call the library")

    monkeypatch.setattr(cache_mod, "lib", no_launch)
    layers = [Layer(SCALES), Layer(SCALES)]
    for layer in layers:
        assert arm(layer, Method(layer, reads=SCALE_NAMES))[0]
    a, b = (layer._expert_cache for layer in layers)
    pred = torch.zeros(2, dtype=torch.int32)
    assert b.prefetch(pred, along=a) is True
    assert a._rider[0] is b and b._riding_on is a
    assert a._rider[2] == b.S  # budget defaults to S
    # a prediction wider than the slots is refused before anything is staged or launched
    assert a.prefetch(torch.zeros(a.S + 1, dtype=torch.int32), along=b) is False
    assert b._rider is None and a._riding_on is None
    with pytest.raises(ValueError):
        a.prefetch(pred, along=a)
    small = cache_mod.ExpertSlotCache(layers[0], ["w13_weight"], a.E, a.S - 1, "cpu")
    with pytest.raises(ValueError):
        small.prefetch(pred, along=a)
