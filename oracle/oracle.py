"""ctypes binding of the CPU oracle (oracle/policy.c) for numpy arrays.

TEST INFRASTRUCTURE ONLY. tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
compare results against it, or time it as the CPU baseline; the product package never
imports it.

State layout and cold/warm starts follow the reference:
  cold start  vllm_expert_cache/cache.py:84-92   (table=-1, map_cold=arange, slot_expert=-1)
  warm start  tests/test_policy.py:57-76          (hot experts installed in slot order, stamp 0)
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libexpertcache_ref.so")

_LIB = None

_P = ctypes.c_void_p
_I = ctypes.c_int


def lib():
    """Load liboracle.so (built by `make -C oracle`)."""
    global _LIB
    if _LIB is None:
        if not os.path.isfile(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
        h = ctypes.CDLL(LIB_PATH)
        manage_args = [_P, _I, _I, _I, _I, _I] + [_P] * 8 + [_I, _I]
        for name in ("oracle_manage_serial", "oracle_manage_rank"):
            f = getattr(h, name)
            f.restype = _I
            f.argtypes = manage_args
        h.oracle_remap_i32.restype = None
        h.oracle_remap_i32.argtypes = [_P, _I, _P, _I, _P]
        h.oracle_remap_i64.restype = None
        h.oracle_remap_i64.argtypes = [_P, _I, _P, _I, _P]
        h.oracle_gather.restype = None
        h.oracle_gather.argtypes = [_I, _P, _P, _P, _P, _I]
        h.oracle_run_trace.restype = _I
        h.oracle_run_trace.argtypes = [_P, _I, _I, _I, _I, _I, _I, _I] + [_P] * 11
        h.oracle_now.restype = ctypes.c_double
        h.oracle_now.argtypes = []
        h.oracle_prefetch.restype = _I
        h.oracle_prefetch.argtypes = [_P, _I, _I, _I, _I] + [_P] * 7 + [_I]
        h.oracle_fused.restype = _I
        h.oracle_fused.argtypes = ([_P, _I, _I, _I, _I, _I] + [_P] * 8 + [_I, _I, _I]
                                   + [_P] * 6)
        h.oracle_fused_trace.restype = _I
        h.oracle_fused_trace.argtypes = [_P] + [_I] * 7 + [_P] * 14
        _LIB = h
    return _LIB


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


class State:
    """One layer's cache state as numpy arrays, laid out as the device tensors are."""

    FIELDS = ("table", "map_cold", "slot_expert", "slot_stamp", "routed", "step", "miss",
              "n_miss")

    def __init__(self, E: int, S: int, hot=None, miss_cap: int | None = None):
        self.E, self.S = int(E), int(S)
        self.table = np.full(E, -1, np.int32)
        self.map_cold = np.arange(E, dtype=np.int32)
        self.slot_expert = np.full(S, -1, np.int32)
        self.slot_stamp = np.zeros(S, np.int64)
        self.routed = np.zeros(E, np.uint8)
        self.step = np.zeros(1, np.int64)
        self.miss = np.zeros(2 * (S if miss_cap is None else miss_cap), np.int32)
        self.n_miss = np.zeros(1, np.int32)
        if hot is not None:
            hot = np.asarray(hot, dtype=np.int64)
            self.table[hot] = np.arange(len(hot), dtype=np.int32)
            self.map_cold[hot] = -1
            self.slot_expert[: len(hot)] = hot.astype(np.int32)

    def copy(self) -> "State":
        c = State.__new__(State)
        c.E, c.S = self.E, self.S
        for f in self.FIELDS:
            setattr(c, f, getattr(self, f).copy())
        return c

    def manage(self, ids, max_distinct: int, max_inserts: int, policy: int, decay: int,
               rule: str = "rank") -> int:
        ids = np.ascontiguousarray(np.asarray(ids).ravel().astype(np.int32))
        f = lib().oracle_manage_rank if rule == "rank" else lib().oracle_manage_serial
        return f(_ptr(ids), int(ids.size), self.E, self.S, int(max_distinct),
                 int(max_inserts), _ptr(self.table), _ptr(self.map_cold),
                 _ptr(self.slot_expert), _ptr(self.slot_stamp), _ptr(self.routed),
                 _ptr(self.step), _ptr(self.miss), _ptr(self.n_miss), int(policy), int(decay))

    def prefetch(self, ids, max_inserts: int, rule: str = "rank") -> int:
        """Install-only step for predicted ids (stamp 0, step and hit stamps untouched)."""
        ids = np.ascontiguousarray(np.asarray(ids).ravel().astype(np.int32))
        return lib().oracle_prefetch(
            _ptr(ids), int(ids.size), self.E, self.S, int(max_inserts), _ptr(self.table),
            _ptr(self.map_cold), _ptr(self.slot_expert), _ptr(self.slot_stamp),
            _ptr(self.routed), _ptr(self.miss), _ptr(self.n_miss), 0 if rule == "serial" else 1)

    def fused(self, ids, max_distinct: int, max_inserts: int, bs: int, L: int, NB: int):
        ids = np.ascontiguousarray(np.asarray(ids).ravel().astype(np.int32))
        out = {k: np.zeros(n, np.int32) for k, n in
               (("sorted_hot", L), ("eids_hot", NB), ("npad_hot", 1),
                ("sorted_cold", L), ("eids_cold", NB), ("npad_cold", 1))}
        rc = lib().oracle_fused(
            _ptr(ids), int(ids.size), self.E, self.S, int(max_distinct), int(max_inserts),
            _ptr(self.table), _ptr(self.map_cold), _ptr(self.slot_expert),
            _ptr(self.slot_stamp), _ptr(self.routed), _ptr(self.step), _ptr(self.miss),
            _ptr(self.n_miss), int(bs), int(L), int(NB),
            *[_ptr(out[k]) for k in ("sorted_hot", "eids_hot", "npad_hot", "sorted_cold",
                                     "eids_cold", "npad_cold")])
        return rc, out

    def fused_trace(self, ids, bs: int, L: int, NB: int) -> int:
        """fused over every row of ids[T, mk] (max_distinct = min(E, mk), max_inserts = S) in
        one C loop; the align outputs are discarded. For timing."""
        ids = np.ascontiguousarray(np.asarray(ids).astype(np.int32))
        T, mk = ids.shape
        out = [np.zeros(n, np.int32) for n in (L, NB, 1, L, NB, 1)]
        return lib().oracle_fused_trace(
            _ptr(ids), T, mk, self.E, self.S, int(bs), int(L), int(NB), _ptr(self.table),
            _ptr(self.map_cold), _ptr(self.slot_expert), _ptr(self.slot_stamp),
            _ptr(self.routed), _ptr(self.step), _ptr(self.miss), _ptr(self.n_miss),
            *[_ptr(o) for o in out])

    def misses(self):
        n = int(self.n_miss[0])
        return [(int(self.miss[2 * j]), int(self.miss[2 * j + 1])) for j in range(n)]


def state_words(E: int, S: int) -> int:
    """int32 words per recorded state: table | map_cold | slot_expert | slot_stamp | step."""
    return 2 * E + 3 * S + 2


def run_trace(ids: np.ndarray, E: int, S: int, policy: int, decay: int = 64,
              rule: str = "rank", state: State | None = None, record_miss: bool = False,
              record_state: bool = False) -> dict:
    """Drive one layer over a trace `ids[T, mk]` the way the plugin does: a step with
    mk > S reads through without calling manage; otherwise max_distinct = min(E, mk) and
    max_inserts = S (vllm_expert_cache/cache.py:99-106, :118-131)."""
    ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int32))
    T, mk = ids.shape
    st = state if state is not None else State(E, S)
    nm = np.zeros(T, np.int32)
    mh = np.zeros((T, 2 * S), np.int32) if record_miss else None
    sh = np.zeros((T, state_words(E, S)), np.int32) if record_state else None
    rc = lib().oracle_run_trace(
        _ptr(ids), T, mk, E, S, int(policy), int(decay), 0 if rule == "serial" else 1,
        _ptr(st.table), _ptr(st.map_cold), _ptr(st.slot_expert), _ptr(st.slot_stamp),
        _ptr(st.routed), _ptr(st.step), _ptr(st.miss), _ptr(st.n_miss), _ptr(nm),
        _ptr(mh) if mh is not None else None, _ptr(sh) if sh is not None else None)
    if rc != 0:
        raise ValueError(f"oracle_run_trace rc={rc}")
    return {"n_miss": nm, "miss": mh, "state": sh, "final": st}


def remap(ids: np.ndarray, table: np.ndarray) -> np.ndarray:
    """table[ids] with torch's negative wrap, in the dtype of `ids` (int32 or int64)."""
    ids = np.ascontiguousarray(ids)
    table = np.ascontiguousarray(table, dtype=np.int32)
    out = np.empty_like(ids)
    if ids.dtype == np.int32:
        lib().oracle_remap_i32(_ptr(ids), int(ids.size), _ptr(table), int(table.size),
                               _ptr(out))
    elif ids.dtype == np.int64:
        lib().oracle_remap_i64(_ptr(ids), int(ids.size), _ptr(table), int(table.size),
                               _ptr(out))
    else:
        raise TypeError(ids.dtype)
    return out


def gather(dsts, srcs, bytes_per_expert, miss: np.ndarray, n_miss: int) -> None:
    """Byte copy of every (expert, slot) pair in the miss list, per buffer (uint8 arrays)."""
    nb = len(dsts)
    dp = (ctypes.c_void_p * nb)(*[d.ctypes.data for d in dsts])
    sp = (ctypes.c_void_p * nb)(*[s.ctypes.data for s in srcs])
    by = np.ascontiguousarray(np.asarray(bytes_per_expert, dtype=np.int64))
    miss = np.ascontiguousarray(miss, dtype=np.int32)
    lib().oracle_gather(nb, ctypes.cast(dp, ctypes.c_void_p), ctypes.cast(sp, ctypes.c_void_p),
                        _ptr(by), _ptr(miss), int(n_miss))


def now() -> float:
    return lib().oracle_now()
