"""Shared GPU-test machinery: device state laid out per layer, trace drivers for the product
library and for the reference library built from source (oracle/_ref), pinned host memory.

Trace drivers record, without any host sync inside the trace, after every step:
n_miss [T, L], the miss buffer [T, L, 2S], the full state [T, L, words] in the oracle's
word layout (table | map_cold | slot_expert | slot_stamp | step), and, for the fused
remap entry point, the slot ids [T, L, mk].
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

import oracle
from vllm_expert_cache import _lib

DEV = "cuda:0"
P = ctypes.c_void_p


def ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def lib():
    return _lib.lib()


_REF = None


def ref_lib():
    """The reference's own kernels, compiled from kernels/expert_cache.hip into oracle/_ref."""
    global _REF
    if _REF is None:
        if not os.path.isfile(oracle.REF_LIB_PATH):
            return None
        h = ctypes.CDLL(oracle.REF_LIB_PATH)
        for name in ("expert_cache_manage", "expert_cache_gather", "expert_cache_fused"):
            getattr(h, name).restype = ctypes.c_int
            getattr(h, name).argtypes = _lib.SIGNATURES[name]
        _REF = h
    return _REF


class Layers:
    """State of L layers, one row per layer, so one copy per field snapshots all layers."""

    def __init__(self, L: int, E: int, S: int, miss_cap: int | None = None, hot=None):
        self.L, self.E, self.S = L, E, S
        cap = S if miss_cap is None else miss_cap
        i32, i64 = torch.int32, torch.int64
        self.table = torch.full((L, E), -1, dtype=i32, device=DEV)
        self.map_cold = torch.arange(E, dtype=i32, device=DEV).repeat(L, 1)
        self.slot_expert = torch.full((L, S), -1, dtype=i32, device=DEV)
        self.slot_stamp = torch.zeros((L, S), dtype=i64, device=DEV)
        self.routed = torch.zeros((L, E), dtype=torch.uint8, device=DEV)
        self.step = torch.zeros((L, 1), dtype=i64, device=DEV)
        self.miss = torch.zeros((L, 2 * cap), dtype=i32, device=DEV)
        self.n_miss = torch.zeros((L, 1), dtype=i32, device=DEV)
        if hot is not None:
            h = torch.as_tensor(hot, dtype=torch.int64, device=DEV)
            self.table[:, h] = torch.arange(len(hot), dtype=i32, device=DEV)
            self.map_cold[:, h] = -1
            self.slot_expert[:, :len(hot)] = h.to(i32)

    def row(self, name: str, l: int) -> ctypes.c_void_p:
        t = getattr(self, name)
        return ctypes.c_void_p(t.data_ptr() + l * t.stride(0) * t.element_size())

    def state_words(self) -> torch.Tensor:
        """[L, words] int32 in the oracle's layout."""
        return torch.cat([self.table, self.map_cold, self.slot_expert,
                          self.slot_stamp.view(torch.int32), self.step.view(torch.int32)], 1)


def manage_call(h, st: Layers, l: int, ids_ptr, mk: int, md: int, mi: int, policy: int,
                decay: int, out_ptr=None, id_bytes: int = 4):
    common = (st.row("table", l), st.row("map_cold", l), st.row("slot_expert", l),
              st.row("slot_stamp", l), st.row("routed", l), st.row("step", l),
              st.row("miss", l), st.row("n_miss", l), policy, decay)
    if out_ptr is None:
        return h.expert_cache_manage(ids_ptr, mk, st.E, st.S, md, mi, *common, stream())
    return h.expert_cache_manage_remap(ids_ptr, id_bytes, mk, st.E, st.S, md, mi, *common,
                                       out_ptr, stream())


def run_trace(h, ids: np.ndarray, E: int, S: int, policy: int, decay: int = 64,
              fused_remap: bool = False, record_state: bool = True, hot=None,
              md: int | None = None, mi: int | None = None, gate: bool = True) -> dict:
    """Drive L layers over ids[T, L, mk] the way the plugin does (a step with mk > S is read
    through without a call; else max_distinct = min(E, mk), max_inserts = S), or, with
    gate=False and explicit md / mi, call manage on every step like the reference's policy
    suites do. Returns numpy histories."""
    T, L, mk = ids.shape
    md = min(E, mk) if md is None else md
    mi = S if mi is None else mi
    st = Layers(L, E, S, miss_cap=mi, hot=hot)
    d_ids = torch.as_tensor(np.ascontiguousarray(ids), device=DEV)
    n_miss = torch.full((T, L), -1, dtype=torch.int32, device=DEV)
    miss = torch.zeros((T, L, 2 * mi), dtype=torch.int32, device=DEV)
    state = (torch.zeros((T, L, oracle.state_words(E, S)), dtype=torch.int32, device=DEV)
             if record_state else None)
    out = torch.full((T, L, mk), -9, dtype=torch.int32, device=DEV) if fused_remap else None
    served = mk <= S or not gate
    row_bytes = mk * 4
    for t in range(T):
        if served:
            for l in range(L):
                ids_ptr = P(d_ids.data_ptr() + (t * L + l) * row_bytes)
                out_ptr = P(out.data_ptr() + (t * L + l) * row_bytes) if fused_remap else None
                rc = manage_call(h, st, l, ids_ptr, mk, md, mi, policy, decay, out_ptr)
                assert rc == 0, rc
            n_miss[t].copy_(st.n_miss[:, 0])
        miss[t].copy_(st.miss)
        if record_state:
            state[t].copy_(st.state_words())
    torch.cuda.synchronize()
    res = {"n_miss": n_miss.cpu().numpy(), "miss": miss.cpu().numpy(), "final": st}
    if record_state:
        res["state"] = state.cpu().numpy()
    if fused_remap:
        res["out"] = out.cpu().numpy()
    return res


def oracle_trace(ids: np.ndarray, E: int, S: int, policy: int, decay: int = 64,
                 record_state: bool = True) -> dict:
    """The oracle over every layer of ids[T, L, mk]; histories shaped like run_trace's."""
    T, L, _ = ids.shape
    nm = np.zeros((T, L), np.int32)
    miss = np.zeros((T, L, 2 * S), np.int32)
    state = np.zeros((T, L, oracle.state_words(E, S)), np.int32) if record_state else None
    finals = []
    for l in range(L):
        r = oracle.run_trace(np.ascontiguousarray(ids[:, l]), E, S, policy, decay,
                             record_miss=True, record_state=record_state)
        nm[:, l] = r["n_miss"]
        miss[:, l] = r["miss"]
        if record_state:
            state[:, l] = r["state"]
        finals.append(r["final"])
    return {"n_miss": nm, "miss": miss, "state": state, "finals": finals}


def first_diff(a: np.ndarray, b: np.ndarray):
    """Index of the first differing element, for failure messages."""
    idx = np.argwhere(a != b)
    return None if len(idx) == 0 else tuple(int(i) for i in idx[0])


def pinned(nbytes: int) -> torch.Tensor:
    """Page-locked host bytes (torch pin_memory allocates them with hipHostMalloc)."""
    return torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)


_HIP = None


def device_pointer(host: torch.Tensor) -> int:
    """Device-side address of pinned host memory (hipHostGetDevicePointer)."""
    global _HIP
    if _HIP is None:
        _HIP = ctypes.CDLL("libamdhip64.so")
        _HIP.hipHostGetDevicePointer.restype = ctypes.c_int
        _HIP.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(ctypes.c_void_p),
                                                 ctypes.c_void_p, ctypes.c_uint]
    dp = ctypes.c_void_p()
    rc = _HIP.hipHostGetDevicePointer(ctypes.byref(dp), ctypes.c_void_p(host.data_ptr()), 0)
    assert rc == 0, f"hipHostGetDevicePointer rc={rc}"
    return dp.value


def fill_random(host: torch.Tensor, seed: int) -> None:
    """Random bytes, generated on the GPU in chunks and copied into `host`."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    chunk = 1 << 28
    for off in range(0, host.numel(), chunk):
        n = min(chunk, host.numel() - off)
        host[off:off + n].copy_(torch.randint(0, 256, (n,), dtype=torch.uint8, device=DEV,
                                              generator=g))
    torch.cuda.synchronize()
