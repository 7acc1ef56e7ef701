"""Arming the slot cache on vLLM MoE layers, whatever the quantisation scheme.

The observable behaviour is the reference's vllm_expert_cache/backends/generic.py:1-361:
which layers are armed, which tensors are mirrored, the log lines, and the keyword
signature of the wrapped `apply`. It is the plugin boundary the accelerated path keeps.

How a layer is served from slots. vLLM's `FusedMoEMethodBase` subclasses share three
habits, and the cache needs nothing else:

  * `apply` reads the expert weights off the layer (layer.w13_weight, layer.w2_weight);
  * `get_fused_moe_quant_config(layer)` rebuilds the per-expert scales, zero points and
    biases by reading layer attributes;
  * the built kernel holds that config in `moe_kernel.fused_experts.quant_config`.

Arming is a plan that either completes or stops with a reason (`_Declined`):

  1. find the expert weight pair, and the slot budget (nothing to do if every expert fits);
  2. refuse layouts the cache cannot serve correctly (`_UNSUPPORTED`);
  3. collect every expert-indexed storage of the layer (`_Mirror`: one storage, every name
     that reaches it), build the cache over them, and decide what each name is rebound to;
  4. ask the method for its config with the layer pointing at the slots, and refuse the
     layer if that config still holds a full [E] tensor (slot ids would index it);
  5. wrap the method's `apply` for this instance only.

A served step applies one `_Patch` (slot tensors, slot config, slot count) around the stock
`apply` and undoes it in reverse order, also when `apply` raises.
"""
from __future__ import annotations

import functools
import sys
from dataclasses import dataclass, field

import torch

from ..cache import ExpertSlotCache
from ..config import settings

# The two expert weight matrices, in the spellings vLLM schemes register: the plain one,
# and the packed compressed-tensors one (wNa16 int4, w4a4 nvfp4 / mxfp4).
_WEIGHT_PAIRS = (("w13_weight", "w2_weight"), ("w13_weight_packed", "w2_weight_packed"))

# Where a FusedMoEQuantConfig keeps per-tensor descriptors, and the descriptor fields that
# can hold a per-expert tensor (vLLM's interface).
_CONFIG_DESCS = ("_a1", "_a2", "_w1", "_w2")
_DESC_TENSORS = ("scale", "alpha_or_gscale", "zp", "bias")

_installed = False


class _Declined(Exception):
    """The layer stays on the stock path. `reason`, when given, is logged as a warning."""

    def __init__(self, reason: str | None = None):
        super().__init__(reason)
        self.reason = reason


# Layouts the cache cannot serve, checked in this order: (test, reason).
_UNSUPPORTED = (
    # apply_monolithic() routes internally: there are no topk_ids to move into slot space
    (lambda layer, m: m.is_monolithic,
     "monolithic method (routing happens inside apply_monolithic)"),
    (lambda layer, m: getattr(m, "moe_kernel", None) is None,
     "method has no moe_kernel (legacy non-modular path)"),
    (lambda layer, m: getattr(m.moe_kernel, "fused_experts", None) is None,
     "moe_kernel exposes no fused_experts to rebind"),
    # with expert parallelism, expert_map folds global ids into a local range; composing it
    # with the slot table would be a second remap
    (lambda layer, m: getattr(layer, "expert_map", None) is not None,
     "expert parallelism active (layer.expert_map is set)"),
)


@dataclass
class _Mirror:
    """One expert-indexed storage of the layer and every attribute name that reaches it, in
    discovery order. The first name is where the cache reads the source from."""

    names: list = field(default_factory=list)

    @property
    def source(self) -> str:
        return self.names[0]


def _is_expert_indexed(value, num_experts: int) -> bool:
    return isinstance(value, torch.Tensor) and value.dim() >= 1 and \
        value.size(0) == num_experts


def _mirrors(layer, num_experts: int) -> list[_Mirror]:
    """Every storage of the layer whose dim 0 is the expert count, with all its names.

    Three registries are read, in this order: registered parameters, registered buffers,
    and plain tensor attributes. The last matters for packed schemes that alias a
    registered tensor under the name `apply` reads (layer.w13_weight =
    layer.w13_weight_packed): both names must be rebound, or apply would keep reading full
    storage with slot ids. Aliases share a storage, so they share one mirror and one slot
    buffer. A dim-0 match that is not really per expert only costs memory; one missed is
    caught by the config check."""
    by_storage: dict[int, _Mirror] = {}
    for registry in (layer._parameters, layer._buffers, vars(layer)):
        for name, value in registry.items():
            if _is_expert_indexed(value, num_experts):
                mirror = by_storage.setdefault(value.data_ptr(), _Mirror())
                if name not in mirror.names:
                    mirror.names.append(name)
    return list(by_storage.values())


def _weight_pair(layer) -> tuple[str, str]:
    for pair in _WEIGHT_PAIRS:
        if all(isinstance(getattr(layer, n, None), torch.Tensor) for n in pair):
            return pair
    registered = sorted(n for n, _ in layer.named_parameters(recurse=False))
    if any("w13" in n or "w2" in n for n in registered):
        # name what is there: a naming convention, not a broken checkpoint
        raise _Declined("no recognised expert weight pair; the layer registers "
                        + (", ".join(registered) or "nothing"))
    raise _Declined()  # not an expert layer this backend knows: nothing to say


def _full_storage_in(cfg, num_experts: int):
    """Descriptor fields of a quant config that still hold a full [E] tensor."""
    for dname in _CONFIG_DESCS:
        desc = getattr(cfg, dname, None)
        for fname in _DESC_TENSORS if desc is not None else ():
            t = getattr(desc, fname, None)
            if _is_expert_indexed(t, num_experts):
                yield f"{dname}.{fname}{tuple(t.shape)}"


def _rebind(layer, name: str, value) -> None:
    """layer.<name> = value, through the registry that holds the name (a bare tensor cannot
    be assigned over a registered Parameter with setattr)."""
    for registry in (layer._parameters, layer._buffers):
        if name in registry:
            registry[name] = value
            return
    setattr(layer, name, value)


class _Patch:
    """Attribute replacements applied one by one and undone in reverse order."""

    __slots__ = ("_undo",)

    def __init__(self):
        self._undo = []

    def set(self, obj, name: str, value) -> None:
        self._undo.append((setattr, obj, name, getattr(obj, name)))
        setattr(obj, name, value)

    def tensor(self, layer, name: str, value) -> None:
        self._undo.append((_rebind, layer, name, getattr(layer, name)))
        _rebind(layer, name, value)

    def slots(self, layer, bound: dict) -> None:
        for name, t in bound.items():
            self.tensor(layer, name, t)

    def undo(self) -> None:
        while self._undo:
            restore, obj, name, old = self._undo.pop()
            restore(obj, name, old)


def _bindings(layer, mirrors: list[_Mirror], slots: dict) -> dict:
    """What each mirrored name points at during a served step: its storage's slot buffer,
    wrapped once as a Parameter for names registered as parameters (graph capture sees
    fixed objects), bare for buffers and plain attributes."""
    bound = {}
    for m in mirrors:
        slot = slots.get(m.source)
        if slot is None:  # not 16-byte aligned per expert: left on full storage
            continue
        as_param = torch.nn.Parameter(slot, requires_grad=False)
        for name in m.names:
            bound[name] = as_param if name in layer._parameters else slot
    return bound


def _plan(layer, method, logger):
    """Steps 1-4 of arming. Returns (cache, config built against the slots)."""
    w13, w2 = _weight_pair(layer)
    num_experts = getattr(layer, w13).size(0)
    slots = settings.slots_for(num_experts)
    if slots >= num_experts:
        raise _Declined()  # every expert fits: slots would only duplicate memory
    for unsupported, reason in _UNSUPPORTED:
        if unsupported(layer, method):
            raise _Declined(reason)

    mirrors = _mirrors(layer, num_experts)
    owner = {name: m for m in mirrors for name in m.names}
    for name in (w13, w2):
        if name not in owner:
            raise _Declined(f"{name} is not a directly-owned expert-major tensor (found: "
                            f"{', '.join(sorted(owner)) or 'none'})")
    try:
        # slots live on the weights' device at load time (the offloader moves the sources
        # to host memory only afterwards)
        cache = ExpertSlotCache(layer, [m.source for m in mirrors], num_experts, slots,
                                getattr(layer, w13).device,
                                required=set(owner[w13].names) | set(owner[w2].names))
    except ValueError as e:  # a weight slab the 16-byte gather cannot move
        raise _Declined(str(e)) from None
    cache.bound = _bindings(layer, mirrors, cache.slots)
    if cache.skipped:
        logger.info("expert-cache: not mirroring %s (not 16-byte aligned per expert); the "
                    "leak check below decides whether that matters", ", ".join(cache.skipped))

    probe = _Patch()
    try:
        probe.slots(layer, cache.bound)
        slot_cfg = method.get_fused_moe_quant_config(layer)
    finally:
        probe.undo()
    leaked = [] if slot_cfg is None else list(_full_storage_in(slot_cfg, num_experts))
    if leaked:
        raise _Declined(f"these per-expert tensors stayed bound to full [{num_experts}] "
                        f"storage after slot binding and would be indexed by slot id: "
                        f"{', '.join(leaked)}")
    return cache, slot_cfg


def _serve_from_slots(layer, method, cache: ExpertSlotCache, slot_cfg) -> None:
    """Step 5: wrap this method instance's apply."""
    stock_apply = method.apply

    # vLLM calls apply by keyword: these parameter names are the contract
    def apply(layer, x, topk_weights, topk_ids, shared_experts=None,
              shared_experts_input=None):
        if not cache.fits(topk_ids):
            # a wide (prefill) step reads through the full tensors on the stock path; a
            # prefetch copy still in flight is joined so no side-stream work outlives it
            cache.join()
            return stock_apply(layer, x, topk_weights, topk_ids, shared_experts,
                               shared_experts_input)
        slot_ids = cache.refresh(topk_ids)
        patch = _Patch()
        try:
            patch.set(method.moe_kernel.fused_experts, "quant_config", slot_cfg)
            patch.set(method, "moe_quant_config", slot_cfg)
            patch.set(layer, "global_num_experts", cache.S)
            patch.slots(layer, cache.bound)
            return stock_apply(layer, x, topk_weights, slot_ids, shared_experts,
                               shared_experts_input)
        finally:
            patch.undo()

    method.apply = apply
    layer._expert_cache = cache


def arm(layer, method, logger) -> bool:
    """Attach a slot cache to one MoE layer. Returns True if the cache is live."""
    try:
        cache, slot_cfg = _plan(layer, method, logger)
    except _Declined as d:
        if d.reason:
            logger.warning("expert-cache: not caching %s -- %s", type(method).__name__,
                           d.reason)
        return False
    _serve_from_slots(layer, method, cache, slot_cfg)
    return True


def _arm_model(model, method_base, logger) -> None:
    """Arm every MoE layer of a loaded model and log one summary line."""
    armed: list = []
    declined = 0
    served_by: set[int] = set()  # method instances already wrapped
    for _, module in model.named_modules():
        method = getattr(module, "quant_method", None)
        if not isinstance(method, method_base):
            continue
        if id(method) in served_by:
            # a method instance shared by two layers would bind its slot config to the
            # first layer's buffers and serve one layer's experts to another
            logger.warning("expert-cache: %s instance is shared across layers; leaving the "
                           "extra layers uncached", type(method).__name__)
            declined += 1
            continue
        try:
            ok = arm(module, method, logger)
        except Exception as e:  # never break serving: the layer reads through as before
            logger.warning("expert-cache: disabled for layer (%r)", e)
            module._expert_cache = None
            ok = False
        if ok:
            served_by.add(id(method))
            armed.append(module._expert_cache)
        else:
            declined += 1
    if not armed:
        logger.info("expert-cache: no cacheable MoE layer found; staying out of the way")
        return
    c = armed[0]
    logger.info("expert-cache %s active on %d MoE layer(s) (%d declined): %d/%d experts "
                "resident, mirroring %s, policy=%s", _version(), len(armed), declined, c.S,
                c.E, "+".join(c.names), settings.policy)


def install(logger) -> bool:
    """Wrap vLLM's post-load hook so that every MoE layer is armed after weights load."""
    global _installed
    if _installed:
        return True
    try:
        from vllm.model_executor.layers.fused_moe.fused_moe_method_base import (
            FusedMoEMethodBase,
        )
        from vllm.model_executor.model_loader import utils as loader_utils
    except Exception as e:
        logger.debug("expert-cache: vLLM MoE interfaces unavailable (%r)", e)
        return False

    original = loader_utils.process_weights_after_loading

    @functools.wraps(original)
    def process_weights_after_loading(model, model_config, target_device):
        original(model, model_config, target_device)
        if not settings.disabled:
            _arm_model(model, FusedMoEMethodBase, logger)

    # Loaders that imported the function by name (base_loader does) hold their own
    # reference: rebind it in every loaded module that has it, and at the source for
    # modules imported later.
    holders = {modname: mod for modname, mod in list(sys.modules.items())
               if mod is not None and
               getattr(mod, "process_weights_after_loading", None) is original}
    for mod in holders.values():
        mod.process_weights_after_loading = process_weights_after_loading
    loader_utils.process_weights_after_loading = process_weights_after_loading
    logger.info("expert-cache: hooked the MoE loader in %s",
                ", ".join(n.rsplit(".", 1)[-1] for n in holders) or "utils")
    _installed = True
    return True


def _version() -> str:
    from .. import __version__

    return __version__
