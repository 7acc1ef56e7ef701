"""Device-side expert cache for vLLM MoE models, for MI355X (gfx950).

Keeps a bounded set of each MoE layer's experts resident in HBM slots and streams the rest
from host memory, so a mixture-of-experts model larger than the GPU still decodes close to
fully-resident speed. vLLM loads it through the `vllm.general_plugins` entry point
`expert_cache = vllm_expert_cache:install`; `EXPERT_CACHE_DISABLE=1` turns it off.

Drop-in for the reference plugin's surface (vllm_expert_cache/__init__.py:1-38): same
module names, same `install`, `settings` and `__version__`, same environment variables, and
a `libexpertcache.so` with the same C-ABI. The kernels behind it are gfx950-native.
"""
from __future__ import annotations

from .config import settings

__all__ = ["install", "settings"]
__version__ = "0.2.0"


def install() -> None:
    """vLLM plugin hook: arm the cache on every MoE layer once weights are loaded."""
    # vLLM attaches handlers only under "vllm.*", so the logger lives in that tree.
    try:
        from vllm.logger import init_logger

        logger = init_logger("vllm.expert_cache")
    except Exception:  # vLLM absent: plain logging under the same name
        import logging

        logger = logging.getLogger("vllm.expert_cache")

    if settings.disabled:
        logger.info("expert-cache: disabled by EXPERT_CACHE_DISABLE")
        return

    from .backends import generic

    if not generic.install(logger):
        logger.info("expert-cache: could not hook vLLM's MoE loader; staying out of the way")
