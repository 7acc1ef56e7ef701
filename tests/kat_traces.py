"""Routing traces behind the reference's published policy miss counts.

The reference's harness (tests/compare_policies.py:31-93) drives a cold cache, E=128,
top-8, 600 steps, with numpy `default_rng(1234)` re-seeded for every slot budget, and
publishes the insert counts (README.md:177-184, docs/results.md:60-67). These functions
regenerate the same traces with numpy's Generator, following the steps of its two
generators:

  zipf       tests/compare_policies.py:50-55  one skewed stream over a random permutation
  interleave tests/compare_policies.py:58-72  4 tasks round-robin, each a shared half plus
                                              its own draw, skew applied by pool position

They are test inputs; the published counts are the expected outputs.
"""
from __future__ import annotations

import numpy as np

E, TOP_K, STEPS, SEED = 128, 8, 600, 1234

# insert counts (LRU, LFU) per (workload, slots), README.md:177-184
KAT = {
    ("zipf", 16): (2392, 1980),
    ("zipf", 32): (1555, 1239),
    ("zipf", 64): (758, 674),
    ("interleave", 16): (2289, 1899),
    ("interleave", 32): (1347, 1096),
    ("interleave", 64): (489, 363),
}


def _zipf_weights(n: int, a: float) -> np.ndarray:
    w = np.arange(1, n + 1, dtype=np.float64) ** (-a)
    return w / w.sum()


def zipf(rng: np.random.Generator, steps: int = STEPS, n: int = E, k: int = TOP_K,
         a: float = 1.2) -> np.ndarray:
    w = _zipf_weights(n, a)
    perm = rng.permutation(n)
    return np.stack([perm[rng.choice(n, size=k, replace=False, p=w)] for _ in range(steps)])


def interleave(rng: np.random.Generator, steps: int = STEPS, n: int = E, k: int = TOP_K,
               ntask: int = 4, a: float = 1.2, shared: float = 0.5) -> np.ndarray:
    w = _zipf_weights(n, a)
    nshare = int(n * shared)
    common = rng.permutation(n)[:nshare]
    pools = [np.concatenate([common, rng.permutation(n)[:n - nshare]]) for _ in range(ntask)]
    rows = []
    for i in range(steps):
        pool = pools[i % ntask]
        p = w[:len(pool)] / w[:len(pool)].sum()
        rows.append(pool[rng.choice(len(pool), size=k, replace=False, p=p)])
    return np.stack(rows)


def trace(workload: str) -> np.ndarray:
    """The [600, 8] int32 trace for one workload (the seed is the same for every budget)."""
    gen = zipf if workload == "zipf" else interleave
    return gen(np.random.default_rng(SEED)).astype(np.int32)
