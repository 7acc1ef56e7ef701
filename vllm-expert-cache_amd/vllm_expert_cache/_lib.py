"""ctypes binding of libexpertcache.so (C-ABI in include/expert_cache.h).

Same search order and same argument lists for the reference's two bound entry points
(vllm_expert_cache/_lib.py:15-61): manage and gather. Six more are bound here:
`expert_cache_fused` (exported by the reference but never bound), the two remap entry
points that replace the reference's torch remap, `expert_cache_prefetch`,
`expert_cache_manage_remap_prefetch` (one layer's policy step with another's prefetch step
in one launch), and `expert_cache_gather_live` (the prefetch copy that stops for dropped
predictions). Every call is asynchronous on the caller's stream and never reads a device
value back, so the whole path is HIP-graph capturable.

There is no fallback: if the library or one of its symbols is missing, loading fails with
an error that says so.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

_LIB = None

_SEARCH = (
    lambda: os.environ.get("EXPERT_CACHE_LIB"),
    lambda: str(Path(__file__).parent / "libexpertcache.so"),
    lambda: "/usr/local/lib/libexpertcache.so",
)

_P, _I, _L = ctypes.c_void_p, ctypes.c_int, ctypes.c_long

# entry point -> argtypes; every restype is int (0 ok, -1 bad arguments, else hipError_t)
SIGNATURES = {
    # manage(ids, mk, E, S, max_distinct, max_inserts, table, map_cold, slot_expert,
    #        slot_stamp, routed, step, miss, n_miss, policy, decay, stream)
    "expert_cache_manage": [_P] + [_I] * 5 + [_P] * 8 + [_I] * 2 + [_P],
    # gather(6 x (dst, src, bytes_per_expert), miss, n_miss, chunks, lanes, stream)
    "expert_cache_gather": [_P, _P, _L] * 6 + [_P, _P, _I, _I, _P],
    # gather_live(6 x (dst, src, bytes_per_expert), miss, n_miss, slot_expert, chunks, lanes,
    #             stream)
    "expert_cache_gather_live": [_P, _P, _L] * 6 + [_P, _P, _P, _I, _I, _P],
    # fused(manage args without policy/decay, bs, L, NB, sorted_hot, eids_hot, npad_hot,
    #       sorted_cold, eids_cold, npad_cold, stream)
    "expert_cache_fused": [_P] + [_I] * 5 + [_P] * 8 + [_I] * 3 + [_P] * 6 + [_P],
    # remap(ids, n, id_bytes, table, E, out, stream)
    "expert_cache_remap": [_P, _I, _I, _P, _I, _P, _P],
    # manage_remap(ids, id_bytes, mk, E, S, max_distinct, max_inserts, table, map_cold,
    #              slot_expert, slot_stamp, routed, step, miss, n_miss, policy, decay, out,
    #              stream)
    "expert_cache_manage_remap": [_P] + [_I] * 6 + [_P] * 8 + [_I] * 2 + [_P, _P],
    # prefetch(pred_ids, mk, E, S, max_inserts, table, map_cold, slot_expert, slot_stamp,
    #          routed, miss, n_miss, stream)
    "expert_cache_prefetch": [_P] + [_I] * 4 + [_P] * 7 + [_P],
    # manage_remap_prefetch(manage_remap args without stream, pred_ids, pk, pf_max_inserts,
    #                       pf_table, pf_map_cold, pf_slot_expert, pf_slot_stamp, pf_routed,
    #                       pf_miss, pf_n_miss, stream)
    "expert_cache_manage_remap_prefetch": ([_P] + [_I] * 6 + [_P] * 8 + [_I, _I, _P]
                                           + [_P, _I, _I] + [_P] * 7 + [_P]),
}


def library_path() -> str:
    for probe in _SEARCH:
        p = probe()
        if p and Path(p).is_file():
            return p
    raise FileNotFoundError(
        "libexpertcache.so not found. Build it for gfx950 with "
        "`python vllm-expert-cache_amd/build.py` (it lands next to this package) or point "
        "EXPERT_CACHE_LIB at it.")


def bind(handle: ctypes.CDLL) -> ctypes.CDLL:
    """Set restype/argtypes of every entry point; raise if one is not exported."""
    missing = [name for name in SIGNATURES if not hasattr(handle, name)]
    if missing:
        raise RuntimeError(f"{handle._name} does not export {', '.join(missing)}")
    for name, argtypes in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = ctypes.c_int
        fn.argtypes = argtypes
    return handle


def lib() -> ctypes.CDLL:
    """Load and bind the kernel library once per process."""
    global _LIB
    if _LIB is None:
        _LIB = bind(ctypes.CDLL(library_path()))
    return _LIB


# The gather entry point copies a fixed six per-expert buffers per call. Callers with fewer
# pad by repeating a buffer they already pass (copied once: the library skips repeats);
# every slab must be a multiple of 16 bytes and dst/src must agree on bytes per expert.
GATHER_SLOTS = 6
