"""Arming logic of backends/generic.py on the CPU, against stand-ins for vLLM's MoE classes.

The situations the reference checks (tests/test_generic.py:142-352): which tensors are
mirrored, that a served step sees slot storage and a slot-sized config, that a wide step
reads through, that the keyword call works, that the layer is restored, and that every
unsafe layout is refused with a reason. Beyond those: the loader hook that `install`
places, driven through a stand-in vLLM module tree (rebinding in modules that imported the
hook by name, arming a model, shared method instances, a layer whose arming raises, and
EXPERT_CACHE_DISABLE).

`refresh` is replaced by an identity, so only the binding is under test; the kernels are
covered by the GPU tests.
"""
from __future__ import annotations

import logging
import sys
import types

import pytest
import torch

from vllm_expert_cache.backends import generic

E, S = 16, 4
HID, INTER = 8, 12


@pytest.fixture(autouse=True)
def _budget(monkeypatch):
    monkeypatch.setenv("EXPERT_CACHE_SLOTS", str(S))
    monkeypatch.delenv("EXPERT_CACHE_DISABLE", raising=False)
    torch.manual_seed(0)


class Captured(logging.Handler):
    """A logger whose formatted messages the test can search."""

    def __init__(self, name):
        super().__init__(logging.DEBUG)
        self.lines: list[str] = []
        self.logger = logging.getLogger(name)
        self.logger.handlers = [self]
        self.logger.setLevel(logging.DEBUG)
        self.logger.propagate = False

    def emit(self, record):
        self.lines.append(record.getMessage())

    def has(self, text: str) -> bool:
        return any(text in line for line in self.lines)


def new_log(tag="t") -> Captured:
    return Captured(f"test.expert_cache.{tag}")


# ---- stand-ins for vLLM's MoE objects -----------------------------------------------------

def quant_config(w1=None, w2=None, w1_zp=None, w2_zp=None, w1_bias=None):
    """A FusedMoEQuantConfig-shaped object: descriptors _a1, _a2, _w1, _w2, each with the
    scale / alpha_or_gscale / zp / bias fields."""
    def desc(scale=None, zp=None, bias=None):
        return types.SimpleNamespace(scale=scale, alpha_or_gscale=None, zp=zp, bias=bias)
    return types.SimpleNamespace(_a1=desc(), _a2=desc(), _w1=desc(w1, w1_zp, w1_bias),
                                 _w2=desc(w2, w2_zp))


def moe_layer(experts=E, **extra) -> torch.nn.Module:
    """A FusedMoE-like module: expert tensors registered as parameters. `extra` maps a
    name to the shape of another parameter."""
    layer = torch.nn.Module()
    frozen = {"requires_grad": False}
    layer.register_parameter("w13_weight",
                             torch.nn.Parameter(torch.randn(experts, INTER, HID), **frozen))
    layer.register_parameter("w2_weight",
                             torch.nn.Parameter(torch.randn(experts, HID, INTER // 2), **frozen))
    for name, shape in extra.items():
        layer.register_parameter(name, torch.nn.Parameter(torch.randn(*shape), **frozen))
    layer.global_num_experts = experts
    layer.expert_map = None
    return layer


class MoEMethod:
    """A FusedMoEMethodBase-like method. Its config factory reads the layer attributes named
    in `scales` (w1 scale, w2 scale, w1 zero point, w2 zero point, in that order); `hidden`
    is a per-expert tensor the factory adds on its own, which no layer attribute reaches.
    Every apply call is recorded in `calls`."""

    is_monolithic = False

    def __init__(self, layer, scales=(), hidden=None):
        self.scales, self.hidden = tuple(scales), hidden
        self.moe_quant_config = self.get_fused_moe_quant_config(layer)
        self.moe_kernel = types.SimpleNamespace(
            fused_experts=types.SimpleNamespace(quant_config=self.moe_quant_config))
        self.calls: list[dict] = []

    def get_fused_moe_quant_config(self, layer):
        got = dict(zip(("w1", "w2", "w1_zp", "w2_zp"),
                       (getattr(layer, n) for n in self.scales)))
        return quant_config(w1_bias=self.hidden, **got)

    def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None,
              shared_experts_input=None):
        self.calls.append({"w13": layer.w13_weight, "w2": layer.w2_weight,
                           "config": self.moe_kernel.fused_experts.quant_config,
                           "ids": topk_ids.clone(), "experts": layer.global_num_experts})
        return torch.zeros(1)


SCALES = {"w13_weight_scale": (E, INTER, 1), "w2_weight_scale": (E, HID, 1)}
ZEROS = {"w13_weight_zero_point": (E, INTER, 1), "w2_weight_zero_point": (E, HID, 1)}


def armed(layer, method, tag="t"):
    log = new_log(tag)
    return generic.arm(layer, method, log.logger), log


def identity_refresh(layer):
    layer._expert_cache.refresh = lambda ids: ids.clone()


def decode_step(method, layer, n_ids=2):
    return method.apply(layer, torch.randn(1, HID), torch.ones(1, n_ids),
                        torch.zeros(1, n_ids, dtype=torch.int32))


# ---- which tensors are mirrored -----------------------------------------------------------

def test_unquantized_layer_mirrors_its_two_weights():
    layer = moe_layer()
    ok, _ = armed(layer, MoEMethod(layer))
    assert ok and sorted(layer._expert_cache.names) == ["w13_weight", "w2_weight"]


def test_int8_layer_mirrors_weights_and_scales():
    layer = moe_layer(**SCALES)
    ok, _ = armed(layer, MoEMethod(layer, scales=SCALES))
    assert ok
    assert sorted(layer._expert_cache.names) == sorted(["w13_weight", "w2_weight", *SCALES])


def test_wna16_layer_mirrors_six_tensors():
    layer = moe_layer(**SCALES, **ZEROS)
    ok, _ = armed(layer, MoEMethod(layer, scales=[*SCALES, *ZEROS]))
    assert ok and len(layer._expert_cache.names) == 6


def test_packed_weights_and_their_aliases_share_one_slot_buffer():
    layer = moe_layer()
    for w in ("w13", "w2"):
        t = layer._parameters.pop(f"{w}_weight")
        layer.register_parameter(f"{w}_weight_packed", t)
        setattr(layer, f"{w}_weight", t)  # the alias apply reads (a second registration)
    method = MoEMethod(layer)
    ok, log = armed(layer, method)
    assert ok, log.lines
    cache = layer._expert_cache
    assert len(cache.slots) == 2
    assert sorted(cache.bound) == ["w13_weight", "w13_weight_packed", "w2_weight",
                                   "w2_weight_packed"]
    assert cache.bound["w13_weight"].data_ptr() == cache.bound["w13_weight_packed"].data_ptr()
    identity_refresh(layer)
    decode_step(method, layer)
    assert method.calls[-1]["w13"].data_ptr() == cache.slots["w13_weight_packed"].data_ptr()
    assert layer.w13_weight.data_ptr() == layer.w13_weight_packed.data_ptr()


class RecordsAliases(MoEMethod):
    """Records where a buffer and a plain tensor attribute point during apply."""

    def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None,
              shared_experts_input=None):
        self.calls.append({"buffer": layer.w13_input_scale.data_ptr(),
                           "attribute": layer.w2_bias.data_ptr()})
        return torch.zeros(1)


def test_buffers_and_plain_attributes_are_mirrored_and_rebound_bare():
    """A per-expert buffer and a plain tensor attribute are mirrored like parameters, and
    rebound bare (not wrapped as Parameters) during a served step."""
    layer = moe_layer()
    layer.register_buffer("w13_input_scale", torch.randn(E, 4))
    layer.w2_bias = torch.randn(E, HID)
    before = (layer.w13_input_scale.data_ptr(), layer.w2_bias.data_ptr())
    method = RecordsAliases(layer)
    ok, _ = armed(layer, method)
    assert ok
    cache = layer._expert_cache
    assert {"w13_input_scale", "w2_bias"} <= set(cache.names)
    assert isinstance(cache.bound["w13_weight"], torch.nn.Parameter)
    assert not isinstance(cache.bound["w13_input_scale"], torch.nn.Parameter)
    assert not isinstance(cache.bound["w2_bias"], torch.nn.Parameter)
    identity_refresh(layer)
    decode_step(method, layer)
    assert method.calls[-1] == {"buffer": cache.slots["w13_input_scale"].data_ptr(),
                                "attribute": cache.slots["w2_bias"].data_ptr()}
    assert (layer.w13_input_scale.data_ptr(), layer.w2_bias.data_ptr()) == before


# ---- served and read-through steps ---------------------------------------------------------

def test_wide_step_reads_through_on_full_storage():
    layer = moe_layer(**SCALES)
    method = MoEMethod(layer, scales=SCALES)
    assert armed(layer, method)[0]
    decode_step(method, layer, n_ids=S + 1)
    call = method.calls[-1]
    assert call["config"]._w1.scale.size(0) == E and call["experts"] == E
    assert call["w13"].data_ptr() == layer.w13_weight.data_ptr()


def test_fitting_step_is_served_from_slots():
    layer = moe_layer(**SCALES)
    method = MoEMethod(layer, scales=SCALES)
    assert armed(layer, method)[0]
    identity_refresh(layer)
    decode_step(method, layer)
    call = method.calls[-1]
    assert call["w13"].data_ptr() == layer._expert_cache.slots["w13_weight"].data_ptr()
    assert call["config"]._w1.scale.size(0) == S and call["experts"] == S


def test_apply_is_called_by_keyword():
    layer = moe_layer()
    method = MoEMethod(layer)
    assert armed(layer, method)[0]
    identity_refresh(layer)
    method.apply(layer=layer, x=torch.randn(1, HID), topk_weights=torch.ones(1, 2),
                 topk_ids=torch.zeros(1, 2, dtype=torch.int32), shared_experts=None,
                 shared_experts_input=None)
    assert len(method.calls) == 1


def test_layer_and_method_are_restored_after_a_step():
    layer = moe_layer(**SCALES)
    method = MoEMethod(layer, scales=SCALES)
    names = ("w13_weight", "w2_weight", *SCALES)
    before = {n: getattr(layer, n).data_ptr() for n in names}
    assert armed(layer, method)[0]
    identity_refresh(layer)
    decode_step(method, layer)
    assert {n: getattr(layer, n).data_ptr() for n in names} == before
    assert layer.global_num_experts == E
    assert method.moe_kernel.fused_experts.quant_config._w1.scale.size(0) == E
    assert method.moe_quant_config._w1.scale.size(0) == E


class FailsInApply(MoEMethod):
    def apply(self, layer, x, topk_weights, topk_ids, shared_experts=None,
              shared_experts_input=None):
        raise RuntimeError("kernel failed")


def test_layer_is_restored_when_apply_raises():
    layer = moe_layer(**SCALES)
    method = FailsInApply(layer, scales=SCALES)
    assert armed(layer, method)[0]
    identity_refresh(layer)
    w13, cfg = layer.w13_weight, method.moe_kernel.fused_experts.quant_config
    with pytest.raises(RuntimeError, match="kernel failed"):
        decode_step(method, layer)
    assert layer.w13_weight is w13 and layer.global_num_experts == E
    assert method.moe_kernel.fused_experts.quant_config is cfg


# ---- layouts that are refused, with a reason -----------------------------------------------

def test_hidden_per_expert_tensor_is_refused():
    layer = moe_layer()
    ok, log = armed(layer, MoEMethod(layer, hidden=torch.randn(E, INTER)))
    assert not ok and log.has("stayed bound to full") and log.has("_w1.bias")
    assert not hasattr(layer, "_expert_cache")


def test_monolithic_method_is_refused():
    layer = moe_layer()
    method = MoEMethod(layer)
    method.is_monolithic = True
    ok, log = armed(layer, method)
    assert not ok and log.has("monolithic")


@pytest.mark.parametrize("strip,needle", [("moe_kernel", "no moe_kernel"),
                                          ("fused_experts", "no fused_experts")])
def test_method_without_a_modular_kernel_is_refused(strip, needle):
    layer = moe_layer()
    method = MoEMethod(layer)
    if strip == "moe_kernel":
        method.moe_kernel = None
    else:
        method.moe_kernel = types.SimpleNamespace(fused_experts=None)
    ok, log = armed(layer, method)
    assert not ok and log.has(needle)


def test_expert_parallel_layer_is_refused():
    layer = moe_layer()
    layer.expert_map = torch.arange(E)
    ok, log = armed(layer, MoEMethod(layer))
    assert not ok and log.has("expert parallelism")


def test_ragged_auxiliary_tensor_is_caught_by_the_config_check():
    layer = moe_layer(w13_weight_scale=(E, 3))  # 12 bytes per expert
    ok, log = armed(layer, MoEMethod(layer, scales=["w13_weight_scale"]))
    assert not ok
    assert log.has("not mirroring w13_weight_scale")
    assert log.has("stayed bound to full") and log.has("w13_weight_scale")


def test_ragged_weight_is_refused():
    layer = moe_layer()
    layer.w13_weight = torch.nn.Parameter(torch.randn(E, 3), requires_grad=False)
    ok, log = armed(layer, MoEMethod(layer))
    assert not ok and log.has("multiple of 16") and log.has("w13_weight")


def test_weight_that_is_not_expert_major_is_refused():
    layer = moe_layer()
    layer.w2_weight = torch.nn.Parameter(torch.randn(HID, E), requires_grad=False)
    ok, log = armed(layer, MoEMethod(layer))
    assert not ok and log.has("w2_weight is not a directly-owned expert-major tensor")


def test_layer_whose_experts_all_fit_is_left_alone(monkeypatch):
    monkeypatch.setenv("EXPERT_CACHE_SLOTS", str(E))
    layer = moe_layer()
    ok, log = armed(layer, MoEMethod(layer))
    assert not ok and log.lines == []


def test_unrecognised_weight_names_are_reported():
    layer = moe_layer()
    layer.register_parameter("w13_qweight", layer._parameters.pop("w13_weight"))
    ok, log = armed(layer, MoEMethod.__new__(MoEMethod))
    assert not ok and log.has("no recognised expert weight pair")
    assert log.has("w13_qweight")


def test_layer_without_expert_weights_is_skipped_silently():
    layer = torch.nn.Module()
    layer.register_parameter("weight", torch.nn.Parameter(torch.randn(4, 4)))
    ok, log = armed(layer, MoEMethod.__new__(MoEMethod))
    assert not ok and log.lines == []


# ---- install() and the loader hook ---------------------------------------------------------

def test_install_without_vllm_stays_out_of_the_way(monkeypatch):
    monkeypatch.setattr(generic, "_installed", False)
    log = new_log("install")
    assert generic.install(log.logger) is False
    assert log.has("vLLM MoE interfaces unavailable")


@pytest.fixture
def fake_vllm(monkeypatch):
    """A stand-in vLLM module tree: the method base class, the loader utils module whose
    process_weights_after_loading is hooked, and a loader module that imported that function
    by name before the plugin was installed."""
    calls = []

    class FusedMoEMethodBase:
        pass

    def process_weights_after_loading(model, model_config, target_device):
        calls.append((model, model_config, target_device))

    tree = {}
    for name in ("vllm", "vllm.model_executor", "vllm.model_executor.layers",
                 "vllm.model_executor.layers.fused_moe",
                 "vllm.model_executor.layers.fused_moe.fused_moe_method_base",
                 "vllm.model_executor.model_loader", "vllm.model_executor.model_loader.utils",
                 "vllm.model_executor.model_loader.base_loader"):
        tree[name] = types.ModuleType(name)
        monkeypatch.setitem(sys.modules, name, tree[name])
    for parent, child in (("vllm", "model_executor"), ("vllm.model_executor", "layers"),
                          ("vllm.model_executor.layers", "fused_moe"),
                          ("vllm.model_executor.layers.fused_moe", "fused_moe_method_base"),
                          ("vllm.model_executor", "model_loader"),
                          ("vllm.model_executor.model_loader", "utils"),
                          ("vllm.model_executor.model_loader", "base_loader")):
        setattr(tree[parent], child, tree[f"{parent}.{child}"])
    tree["vllm.model_executor.layers.fused_moe.fused_moe_method_base"].FusedMoEMethodBase = \
        FusedMoEMethodBase
    tree["vllm.model_executor.model_loader.utils"].process_weights_after_loading = \
        process_weights_after_loading
    tree["vllm.model_executor.model_loader.base_loader"].process_weights_after_loading = \
        process_weights_after_loading
    monkeypatch.setattr(generic, "_installed", False)

    class Method(MoEMethod, FusedMoEMethodBase):
        pass

    return types.SimpleNamespace(tree=tree, calls=calls, Method=Method,
                                 original=process_weights_after_loading)


def _model(method_cls, n_layers=3, share_first_two=False):
    model = torch.nn.Module()
    methods = []
    for i in range(n_layers):
        layer = moe_layer(**SCALES)
        if share_first_two and i == 1:
            layer.quant_method = methods[0]
        else:
            layer.quant_method = method_cls(layer, scales=SCALES)
        methods.append(layer.quant_method)
        model.add_module(f"moe{i}", layer)
    model.add_module("dense", torch.nn.Linear(2, 2))
    return model


def test_install_hooks_every_module_that_holds_the_loader_function(fake_vllm):
    log = new_log("install")
    assert generic.install(log.logger) is True
    utils = fake_vllm.tree["vllm.model_executor.model_loader.utils"]
    base = fake_vllm.tree["vllm.model_executor.model_loader.base_loader"]
    hook = utils.process_weights_after_loading
    assert hook is not fake_vllm.original and base.process_weights_after_loading is hook
    assert hook.__wrapped__ is fake_vllm.original and hook.__name__ == "process_weights_after_loading"
    assert log.has("hooked the MoE loader in") and log.has("base_loader") and log.has("utils")
    assert generic.install(log.logger) is True  # idempotent: no second wrapper
    assert utils.process_weights_after_loading is hook


def test_loader_hook_arms_every_moe_layer_after_loading(fake_vllm):
    log = new_log("hook")
    assert generic.install(log.logger)
    model = _model(fake_vllm.Method)
    hook = fake_vllm.tree["vllm.model_executor.model_loader.base_loader"] \
        .process_weights_after_loading
    hook(model, "cfg", "cuda:7")
    assert fake_vllm.calls == [(model, "cfg", "cuda:7")]  # vLLM's own step ran first
    for i in range(3):
        assert getattr(model, f"moe{i}")._expert_cache is not None
    assert log.has("active on 3 MoE layer(s) (0 declined): 4/16 experts resident, "
                   "mirroring w13_weight+w2_weight+w13_weight_scale+w2_weight_scale, "
                   "policy=lfu")


def test_loader_hook_leaves_a_shared_method_instance_on_one_layer(fake_vllm):
    log = new_log("shared")
    assert generic.install(log.logger)
    model = _model(fake_vllm.Method, share_first_two=True)
    fake_vllm.tree["vllm.model_executor.model_loader.utils"].process_weights_after_loading(
        model, None, None)
    assert hasattr(model.moe0, "_expert_cache") and not hasattr(model.moe1, "_expert_cache")
    assert log.has("instance is shared across layers")
    assert log.has("active on 2 MoE layer(s) (1 declined)")


def test_loader_hook_survives_a_layer_whose_arming_raises(fake_vllm):
    log = new_log("raises")
    assert generic.install(log.logger)
    model = _model(fake_vllm.Method, n_layers=2)

    def explode(layer):
        raise RuntimeError("factory broke")

    model.moe1.quant_method.get_fused_moe_quant_config = explode
    fake_vllm.tree["vllm.model_executor.model_loader.utils"].process_weights_after_loading(
        model, None, None)
    assert model.moe1._expert_cache is None and model.moe0._expert_cache is not None
    assert log.has("disabled for layer") and log.has("factory broke")
    assert log.has("active on 1 MoE layer(s) (1 declined)")


def test_loader_hook_respects_expert_cache_disable(fake_vllm, monkeypatch):
    log = new_log("disabled")
    assert generic.install(log.logger)
    monkeypatch.setenv("EXPERT_CACHE_DISABLE", "1")
    model = _model(fake_vllm.Method, n_layers=1)
    fake_vllm.tree["vllm.model_executor.model_loader.utils"].process_weights_after_loading(
        model, None, None)
    assert not hasattr(model.moe0, "_expert_cache") and len(fake_vllm.calls) == 1


def test_loader_hook_with_no_cacheable_layer_says_so(fake_vllm, monkeypatch):
    log = new_log("none")
    assert generic.install(log.logger)
    monkeypatch.setenv("EXPERT_CACHE_SLOTS", str(E))  # everything fits
    fake_vllm.tree["vllm.model_executor.model_loader.utils"].process_weights_after_loading(
        _model(fake_vllm.Method, n_layers=2), None, None)
    assert log.has("no cacheable MoE layer found")


# ---- host-side prefetch rules that need no kernel -------------------------------------------

def test_prefetch_refuses_a_prediction_wider_than_the_slots():
    """A prediction with more ids than slots is refused before anything is launched, and
    join() with nothing pending does nothing."""
    layer = moe_layer(**SCALES)
    assert armed(layer, MoEMethod(layer, scales=SCALES))[0]
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
    layers = [moe_layer(**SCALES), moe_layer(**SCALES)]
    for layer in layers:
        assert armed(layer, MoEMethod(layer, scales=SCALES))[0]
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
