"""Arming the slot cache on vLLM MoE layers, for any quantisation scheme.

Behaviour follows vllm_expert_cache/backends/generic.py:1-361 of the reference; this is
the boundary the plugin keeps, not part of the accelerated path. It relies on three things
every vLLM `FusedMoEMethodBase` subclass does:

  * `apply` reads the expert weights off the layer (layer.w13_weight, layer.w2_weight);
  * `get_fused_moe_quant_config(layer)` rebuilds the per-expert scales / zero points /
    biases by reading named layer attributes;
  * the built kernel keeps that config in `moe_kernel.fused_experts.quant_config`.

So a cached step points every per-expert attribute at its slot buffer, swaps in a config
built against those buffers, narrows `global_num_experts` to the slot count and calls the
stock `apply` with slot-space ids. Layers the cache cannot serve correctly are declined with
a logged reason and keep running on the stock path.
"""
from __future__ import annotations

import contextlib
import itertools
import sys

import torch

from ..cache import ExpertSlotCache
from ..config import settings

# FusedMoEQuantDesc fields that may hold a per-expert tensor, and the descs of a config
_DESC_FIELDS = ("scale", "alpha_or_gscale", "zp", "bias")
_DESC_NAMES = ("_a1", "_a2", "_w1", "_w2")

_WEIGHT_PAIRS = (("w13_weight", "w2_weight"), ("w13_weight_packed", "w2_weight_packed"))

_installed = False


def _set_tensor(layer, name: str, t: torch.Tensor) -> None:
    """Rebind `layer.<name>` through the registry it lives in (a bare tensor cannot be
    assigned over a registered Parameter)."""
    if name in layer._parameters:
        layer._parameters[name] = t
    elif name in layer._buffers:
        layer._buffers[name] = t
    else:
        setattr(layer, name, t)


def _per_expert_tensors(layer, num_experts: int) -> dict[str, list[str]]:
    """Every expert-indexed storage of the layer (dim 0 == E), with all the names that reach
    it: registered parameters and buffers, and plain tensor attributes. Aliases of one
    storage (`layer.w13_weight = layer.w13_weight_packed`) form one group keyed by its first
    name, so each storage is mirrored once and every alias is rebound."""
    groups: dict[int, list[str]] = {}
    named = itertools.chain(
        # remove_duplicate=False: an aliased Parameter is registered under two names and
        # must be found under both
        layer.named_parameters(recurse=False, remove_duplicate=False),
        layer.named_buffers(recurse=False, remove_duplicate=False),
        ((k, v) for k, v in vars(layer).items() if isinstance(v, torch.Tensor)),
    )
    for name, t in named:
        if not (isinstance(t, torch.Tensor) and t.dim() >= 1 and t.size(0) == num_experts):
            continue
        names = groups.setdefault(t.data_ptr(), [])
        if name not in names:
            names.append(name)
    return {names[0]: names for names in groups.values()}


def _leaked_full_tensors(cfg, num_experts: int) -> list[str]:
    """Per-expert tensors a slot-bound config still takes from full [E] storage. Serving such
    a layer would index expert rows with slot ids -- silently wrong -- so it is declined."""
    leaked = []
    for dname in _DESC_NAMES:
        desc = getattr(cfg, dname, None)
        if desc is None:
            continue
        for field in _DESC_FIELDS:
            t = getattr(desc, field, None)
            if isinstance(t, torch.Tensor) and t.dim() >= 1 and t.size(0) == num_experts:
                leaked.append(f"{dname}.{field}{tuple(t.shape)}")
    return leaked


@contextlib.contextmanager
def _slot_bound(layer, cache: ExpertSlotCache):
    """Point every mirrored attribute at its slot buffer inside the block, then restore."""
    saved = {name: getattr(layer, name) for name in cache.bound}
    try:
        for name, slot in cache.bound.items():
            _set_tensor(layer, name, slot)
        yield
    finally:
        for name, t in saved.items():
            _set_tensor(layer, name, t)


def _decline(layer, method, num_experts: int) -> str | None:
    """Why this layer cannot be cached correctly, or None."""
    if method.is_monolithic:
        return "monolithic method (routing happens inside apply_monolithic)"
    if getattr(method, "moe_kernel", None) is None:
        return "method has no moe_kernel (legacy non-modular path)"
    if getattr(method.moe_kernel, "fused_experts", None) is None:
        return "moe_kernel exposes no fused_experts to rebind"
    if getattr(layer, "expert_map", None) is not None:
        # EP folds global ids into a local range with expert_map; composing that with the
        # slot table is a second remap this cache does not do
        return "expert parallelism active (layer.expert_map is set)"
    return None


def _weight_names(layer) -> tuple[str, str] | None:
    """Registered names of the two expert weight matrices (plain or packed spelling)."""
    for a, b in _WEIGHT_PAIRS:
        if isinstance(getattr(layer, a, None), torch.Tensor) and \
                isinstance(getattr(layer, b, None), torch.Tensor):
            return a, b
    return None


def arm(layer, method, logger) -> bool:
    """Attach a slot cache to one MoE layer. Returns True if the cache is live."""
    names = _weight_names(layer)
    if names is None:
        present = sorted(n for n, _ in layer.named_parameters(recurse=False))
        if any("w13" in n or "w2" in n for n in present):
            logger.warning(
                "expert-cache: not caching %s -- no recognised expert weight pair; the layer "
                "registers %s", type(method).__name__, ", ".join(present) or "nothing")
        return False
    w13_name, w2_name = names

    num_experts = getattr(layer, w13_name).size(0)
    slots = settings.slots_for(num_experts)
    if slots >= num_experts:
        return False  # everything fits already; slots would only duplicate memory

    reason = _decline(layer, method, num_experts)
    if reason is not None:
        logger.warning("expert-cache: not caching %s -- %s", type(method).__name__, reason)
        return False

    sources = _per_expert_tensors(layer, num_experts)
    reachable = {n: key for key, group in sources.items() for n in group}
    for name in (w13_name, w2_name):
        if name not in reachable:
            logger.warning(
                "expert-cache: not caching %s -- %s is not a directly-owned expert-major "
                "tensor (found: %s)", type(method).__name__, name,
                ", ".join(sorted(reachable)) or "none")
            return False
    w13_key, w2_key = reachable[w13_name], reachable[w2_name]

    try:
        cache = ExpertSlotCache(layer, sources.keys(), num_experts, slots,
                                getattr(layer, w13_name).device,
                                required=set(sources[w13_key]) | set(sources[w2_key]))
    except ValueError as e:
        logger.warning("expert-cache: not caching %s -- %s", type(method).__name__, e)
        return False

    # One slot buffer per storage, shared by all its aliases; wrapped as a Parameter once,
    # and only for names registered as parameters.
    cache.bound = {}
    for canonical, group in sources.items():
        if canonical not in cache.slots:
            continue  # not 16-byte aligned: left on full storage for the leak check
        slot = cache.slots[canonical]
        as_param = torch.nn.Parameter(slot, requires_grad=False)
        for name in group:
            cache.bound[name] = as_param if name in layer._parameters else slot

    if cache.skipped:
        logger.info("expert-cache: not mirroring %s (not 16-byte aligned per expert); the "
                    "leak check below decides whether that matters", ", ".join(cache.skipped))

    with _slot_bound(layer, cache):
        slot_cfg = method.get_fused_moe_quant_config(layer)

    if slot_cfg is not None:
        leaked = _leaked_full_tensors(slot_cfg, num_experts)
        if leaked:
            logger.warning(
                "expert-cache: not caching %s -- these per-expert tensors stayed bound to full "
                "[%d] storage after slot binding and would be indexed by slot id: %s",
                type(method).__name__, num_experts, ", ".join(leaked))
            return False

    orig_apply = method.apply

    # vLLM calls apply by keyword, so these parameter names are part of the contract.
    def apply(layer, x, topk_weights, topk_ids, shared_experts=None,
              shared_experts_input=None):
        if not cache.fits(topk_ids):
            # wide (prefill) step: read through the host copies on the stock path; a
            # prefetch still copying is joined so no side-stream work is left behind
            cache.join()
            return orig_apply(layer, x, topk_weights, topk_ids, shared_experts,
                              shared_experts_input)
        slot_ids = cache.refresh(topk_ids)
        experts = method.moe_kernel.fused_experts
        saved = (experts.quant_config, method.moe_quant_config, layer.global_num_experts)
        experts.quant_config = slot_cfg
        method.moe_quant_config = slot_cfg
        layer.global_num_experts = cache.S
        try:
            with _slot_bound(layer, cache):
                return orig_apply(layer, x, topk_weights, slot_ids, shared_experts,
                                  shared_experts_input)
        finally:
            experts.quant_config, method.moe_quant_config, layer.global_num_experts = saved

    method.apply = apply
    layer._expert_cache = cache
    return True


def install(logger) -> bool:
    """Wrap vLLM's post-load hook so every MoE layer is armed after weights load."""
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

    orig = loader_utils.process_weights_after_loading

    def process_weights_after_loading(model, model_config, target_device):
        orig(model, model_config, target_device)
        if settings.disabled:
            return
        armed = declined = 0
        first = None
        seen: set[int] = set()
        for _, module in model.named_modules():
            method = getattr(module, "quant_method", None)
            if not isinstance(method, FusedMoEMethodBase):
                continue
            if id(method) in seen:
                # one method instance serving two layers would bind both to one layer's
                # slots; leave the extra layers uncached
                logger.warning("expert-cache: %s instance is shared across layers; leaving "
                               "the extra layers uncached", type(method).__name__)
                declined += 1
                continue
            try:
                if arm(module, method, logger):
                    armed += 1
                    seen.add(id(method))
                    first = first or module._expert_cache
                else:
                    declined += 1
            except Exception as e:  # never break serving: the layer reads through
                logger.warning("expert-cache: disabled for layer (%r)", e)
                module._expert_cache = None
                declined += 1
        if first is not None:
            logger.info(
                "expert-cache %s active on %d MoE layer(s) (%d declined): %d/%d experts "
                "resident, mirroring %s, policy=%s", _version(), armed, declined, first.S,
                first.E, "+".join(first.names), settings.policy)
        else:
            logger.info("expert-cache: no cacheable MoE layer found; staying out of the way")

    # Rebind in every module that imported the function by name (base_loader does), and
    # at the source for importers not loaded yet.
    patched = []
    for name, mod in list(sys.modules.items()):
        if mod is not None and getattr(mod, "process_weights_after_loading", None) is orig:
            setattr(mod, "process_weights_after_loading", process_weights_after_loading)
            patched.append(name.rsplit(".", 1)[-1])
    loader_utils.process_weights_after_loading = process_weights_after_loading

    logger.info("expert-cache: hooked the MoE loader in %s", ", ".join(patched) or "utils")
    _installed = True
    return True


def _version() -> str:
    from .. import __version__

    return __version__
