"""Runtime configuration: environment variables only, read live on every access.

Names, defaults and parsing follow vllm_expert_cache/config.py:8-47 of the reference, so a
deployment configured for it behaves the same here:

  EXPERT_CACHE_DISABLE   "1" turns the plugin off
  EXPERT_CACHE_SLOTS     absolute slot count (unset or empty: use the fraction)
  EXPERT_CACHE_FRACTION  slots = round(E * fraction) when SLOTS is unset, default 0.5
  EXPERT_CACHE_POLICY    "lfu" (default) or "lru"; any other value means LRU
  EXPERT_CACHE_DECAY     LFU halving period in steps, default 64, 0 = never

EXPERT_CACHE_CHUNKS / EXPERT_CACHE_LANES (gather grid) are read by cache.py and
EXPERT_CACHE_LIB (library path) by _lib.py, as in the reference. EXPERT_CACHE_PREFETCH_CHUNKS
(workgroups of a prefetch copy, default 16) is this package's own, read by cache.py.
"""
from __future__ import annotations

import os

_POLICY_CODES = {"lru": 0, "lfu": 1}


class _Settings:
    @property
    def disabled(self) -> bool:
        return os.environ.get("EXPERT_CACHE_DISABLE", "0") == "1"

    @property
    def slots(self) -> int | None:
        raw = os.environ.get("EXPERT_CACHE_SLOTS")
        return int(raw) if raw else None

    @property
    def fraction(self) -> float:
        return float(os.environ.get("EXPERT_CACHE_FRACTION", "0.5"))

    @property
    def policy(self) -> str:
        return os.environ.get("EXPERT_CACHE_POLICY", "lfu").strip().lower()

    @property
    def policy_code(self) -> int:
        # an unrecognised name silently selects LRU (reference config.py:33-35)
        return _POLICY_CODES.get(self.policy, 0)

    @property
    def decay(self) -> int:
        return int(os.environ.get("EXPERT_CACHE_DECAY", "64"))

    def slots_for(self, num_experts: int) -> int:
        """Slot budget for a layer of `num_experts`: SLOTS, else round(E * FRACTION) with
        Python's half-to-even round, clamped to [1, E]."""
        n = self.slots
        if n is None:
            n = round(num_experts * self.fraction)
        return max(1, min(int(n), num_experts))


settings = _Settings()
