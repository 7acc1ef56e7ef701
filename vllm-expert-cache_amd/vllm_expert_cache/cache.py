"""Per-MoE-layer expert slot cache.

The layer's full expert tensors stay where the offloader put them (host memory the GPU can
read). This class adds `num_slots` HBM slot buffers per mirrored tensor and the device
state of the replacement policy. Each served decode step runs, on the current stream:

  1. expert_cache_manage_remap: marks the routed experts, refreshes their priority, evicts
     the lowest-priority slots this step does not need, installs the missing experts, writes
     the (expert, slot) miss list, and rewrites the routing ids into slot ids -- one
     single-wave kernel.
  2. expert_cache_gather: pulls each missing expert's slabs from host memory into its slot.

The fused-MoE GEMM then runs unchanged against the slot buffers with the slot ids. Nothing
reads a device value back to the host, so the sequence is graph-capturable, and the kernels
are deterministic, so tensor-parallel ranks seeing the same routing keep identical caches
without talking to each other.

A caller that can predict a layer's next routing (for instance from the previous layer's
hidden state) calls `prefetch` early: the install-only policy step runs on the current
stream and the copy of the predicted experts on a side stream, overlapping what follows;
the layer's next `refresh` waits for that copy before its own gather. With `along=` another
layer's cache, the prefetch step waits for that layer's next `refresh` and runs inside the
same launch as its policy step (expert_cache_manage_remap_prefetch), one stream node instead
of two. README.md:392-394 of the reference names prefetch as the path's next step.

Constructor, attributes and methods mirror vllm_expert_cache/cache.py:38-163 of the
reference (`fits`, `remap`, `refresh`, `slots`, `bound`, `names`, `skipped`, `E`, `S`).
"""
from __future__ import annotations

import ctypes
import os

import torch

from ._lib import GATHER_SLOTS, lib
from .config import settings

# Gather grid: chunks x lanes workgroups of 256 lanes, each holding one 8-KB tile of loads
# in flight. The kernel spreads the step's (miss, buffer, tile) work over the whole grid,
# so only the product matters. On MI355X the host link is saturated by ~128-256 KB in
# flight and degrades with much more (measured: 32 workgroups reach ~54.5 GB/s on one
# 4.7 MB expert, 512 reach ~41 GB/s), hence 32 x 1 rather than the reference's 16 x 64.
DEFAULT_CHUNKS = 32
DEFAULT_LANES = 1
# Prefetch copies run beside the decode chain on another stream. The host link is shared
# with the command processor's own reads, so the more a copy keeps in flight, the longer
# every dispatch of the chain waits (measured on MI355X, a dependent 48-layer chain beside a
# streaming copy: +2.4 us per layer at 4 workgroups, +6.7 at 16, +17.5 at 32, +110 at 64,
# while the copy itself reaches 20, 56.7, 57.5 and 56.1 GB/s). 16 workgroups still fill the
# link; in the prefetch pipeline they beat 12, 20, 24 and 32 for every predictor measured.
PREFETCH_CHUNKS = 16

# One side stream per device carries every layer's prefetch copy: the copies share one host
# link, so running them one after another loses nothing. Default priority.
_SIDE: dict = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    if device not in _SIDE:
        _SIDE[device] = torch.cuda.Stream(device)
    return _SIDE[device]


def _bytes_per_expert(t: torch.Tensor) -> int:
    return (t.numel() // t.shape[0]) * t.element_size()


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


_HIP = None


def device_address(t: torch.Tensor) -> int:
    """Address at which the GPU reads `t`: its own for a device tensor (vLLM's offloader
    hands over device views of host memory), or the device mapping of page-locked host
    memory from hipHostGetDevicePointer for a pinned CPU tensor. Pageable memory is refused
    before any HIP call: a failed lookup would leave an error that the next GPU call
    reports."""
    if t.is_cuda:
        return t.data_ptr()
    if not t.is_pinned():
        raise ValueError(f"expert source at {t.data_ptr():#x} is pageable host memory the "
                         f"GPU cannot read; pin it")
    global _HIP
    if _HIP is None:
        _HIP = ctypes.CDLL("libamdhip64.so")
        _HIP.hipHostGetDevicePointer.restype = ctypes.c_int
        _HIP.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(ctypes.c_void_p),
                                                 ctypes.c_void_p, ctypes.c_uint]
        _HIP.hipGetLastError.restype = ctypes.c_int
    out = ctypes.c_void_p()
    rc = _HIP.hipHostGetDevicePointer(ctypes.byref(out), ctypes.c_void_p(t.data_ptr()), 0)
    if rc != 0 or not out.value:
        _HIP.hipGetLastError()  # clear it: the caller gets the error here, not later
        raise ValueError(f"expert source at {t.data_ptr():#x} is host memory the GPU cannot "
                         f"read (hipHostGetDevicePointer rc={rc}); pin it")
    return out.value


class ExpertSlotCache:
    """Holds `num_slots` of `num_experts` experts resident in device memory."""

    def __init__(self, owner, source_names, num_experts: int, num_slots: int, device,
                 required=()):
        # Sources are re-read from `owner` on every step: vLLM's offloader moves expert
        # tensors to host memory after loading, so a pointer taken now would go stale.
        self.owner = owner
        self.names = list(source_names)
        self.E = int(num_experts)
        self.S = int(num_slots)

        # The gather moves 16-byte vectors, so a slab of another size cannot be mirrored. A
        # required one (a weight the GEMM reads directly) is fatal; any other is left
        # unmirrored, and the caller's leak check decides whether the quantisation config
        # actually indexes it per expert.
        fulls = {n: getattr(owner, n).data for n in self.names}
        odd = {n: f"{n}{tuple(t.shape)}={_bytes_per_expert(t)}B" for n, t in fulls.items()
               if _bytes_per_expert(t) % 16}
        fatal = [desc for n, desc in odd.items() if n in required]
        if fatal:
            raise ValueError("per-expert slab must be a multiple of 16 bytes, but these are "
                             "not: " + ", ".join(fatal))
        self.skipped: list[str] = [desc for n, desc in odd.items() if n not in required]
        self.names = [n for n in self.names if n not in odd]
        self.slots: dict[str, torch.Tensor] = {
            n: torch.empty((self.S,) + tuple(fulls[n].shape[1:]), dtype=fulls[n].dtype,
                           device=device) for n in self.names}

        # What the layer's attributes are rebound to during a cached step; built once so
        # graph capture sees fixed storage.
        self.bound: dict[str, torch.Tensor] = dict(self.slots)

        i32, i64, u8 = torch.int32, torch.int64, torch.uint8
        self.table = torch.full((self.E,), -1, dtype=i32, device=device)
        self.map_cold = torch.arange(self.E, dtype=i32, device=device)
        self.slot_expert = torch.full((self.S,), -1, dtype=i32, device=device)
        self.slot_stamp = torch.zeros((self.S,), dtype=i64, device=device)
        self.routed = torch.zeros((self.E,), dtype=u8, device=device)
        self.step = torch.zeros((1,), dtype=i64, device=device)
        self.miss = torch.zeros((2 * self.S,), dtype=i32, device=device)
        self.n_miss = torch.zeros((1,), dtype=i32, device=device)
        # the prefetch step's own miss list: its copy may still read it while the next real
        # step writes `miss`
        self.pf_miss = torch.zeros((2 * self.S,), dtype=i32, device=device)
        self.pf_n_miss = torch.zeros((1,), dtype=i32, device=device)
        self._pf_fork = self._pf_done = None
        self._pf_pending = False
        # prefetch staged to ride with this cache's next policy launch: (cache, ids, budget)
        self._rider = None
        # the cache whose next policy launch carries this cache's staged prefetch
        self._riding_on = None
        # addresses every step passes to the library, fixed for the cache's lifetime (ctypes
        # converts the ints); the gather calls are rebuilt only when a source moves
        self._state = tuple(t.data_ptr() for t in (
            self.table, self.map_cold, self.slot_expert, self.slot_stamp, self.routed,
            self.step, self.miss, self.n_miss))
        self._pf_state = tuple(t.data_ptr() for t in (
            self.table, self.map_cold, self.slot_expert, self.slot_stamp, self.routed,
            self.pf_miss, self.pf_n_miss))
        self._gather_key = None
        self._gather_srcs = ()
        self._gather_calls = ()

        self.policy = settings.policy_code
        self.decay = settings.decay
        self.chunks = int(os.environ.get("EXPERT_CACHE_CHUNKS", str(DEFAULT_CHUNKS)))
        self.lanes = int(os.environ.get("EXPERT_CACHE_LANES", str(DEFAULT_LANES)))
        self.pf_chunks = int(os.environ.get("EXPERT_CACHE_PREFETCH_CHUNKS",
                                            str(PREFETCH_CHUNKS)))

    def fits(self, topk_ids: torch.Tensor) -> bool:
        """Can this step be served from slots? tokens x top_k bounds the distinct experts
        the step touches; it is shape metadata, so deciding costs no device sync."""
        return topk_ids.numel() <= self.S

    @staticmethod
    def _id_view(topk_ids: torch.Tensor) -> tuple[torch.Tensor, int]:
        if topk_ids.dtype == torch.int32:
            return topk_ids.contiguous(), 4
        if topk_ids.dtype == torch.int64:
            return topk_ids.contiguous(), 8
        return topk_ids.to(torch.int32).contiguous(), 4

    def _stream(self) -> ctypes.c_void_p:
        return ctypes.c_void_p(torch.cuda.current_stream(self.table.device).cuda_stream)

    def remap(self, topk_ids: torch.Tensor) -> torch.Tensor:
        """Routing ids rewritten as slot ids against the current table (negative ids wrap
        as torch indexing does). Valid after `refresh`."""
        ids, nbytes = self._id_view(topk_ids)
        out = torch.empty_like(ids)
        rc = lib().expert_cache_remap(_ptr(ids), int(ids.numel()), nbytes, _ptr(self.table),
                                      self.E, _ptr(out), self._stream())
        if rc != 0:
            raise RuntimeError(f"expert_cache_remap failed rc={rc}")
        return out if out.dtype == topk_ids.dtype else out.to(topk_ids.dtype)

    def refresh(self, topk_ids: torch.Tensor) -> torch.Tensor:
        """Run the policy step and the gather for this step; return slot-space ids. A
        prefetch staged with `along=self` runs in the same launch as the policy step."""
        h = lib()
        if self._riding_on is not None:  # this layer's own staged prefetch goes first
            self._riding_on._flush_rider()
        self._plan()  # a source the GPU cannot read is refused before the state changes
        if self._rider is not None:
            self._rider[0]._plan()
        stream = self._stream()
        ids, nbytes = self._id_view(topk_ids)
        out = torch.empty_like(ids)
        mk = int(ids.numel())
        own = (ids.data_ptr(), nbytes, mk, self.E, self.S, min(self.E, mk), self.S,
               *self._state, self.policy, self.decay, out.data_ptr())
        rider = self._rider
        if rider is None:
            rc = h.expert_cache_manage_remap(*own, stream)
        else:
            other, pred, budget = rider
            self._rider = other._riding_on = None
            other._wait_copy()  # its previous copy may still read pf_miss
            rc = h.expert_cache_manage_remap_prefetch(
                *own, pred.data_ptr(), int(pred.numel()), budget, *other._pf_state, stream)
        if rc != 0:
            raise RuntimeError(f"expert_cache_manage failed rc={rc}")
        if rider is not None:
            # forked right after the launch, the copy starts as early as it can; forked after
            # this layer's gather it would share the link less with that gather, but a right
            # prediction leaves that gather empty, and the later start measured slower
            rider[0]._copy_prefetched()
        # a prefetched slot may be this step's victim: its copy lands before this gather
        self._wait_copy()
        self._gather(self.miss, self.n_miss, stream)
        return out if out.dtype == topk_ids.dtype else out.to(topk_ids.dtype)

    def prefetch(self, pred_ids: torch.Tensor, max_inserts: int | None = None,
                 along: "ExpertSlotCache | None" = None) -> bool:
        """Start bringing the experts predicted for this layer's next step into slots.

        The prefetch policy step (expert_cache_prefetch: pending installs, no step
        advance, resident predictions untouched, at most `max_inserts` installs, which
        defaults to S and is capped there) runs on the current stream. The copy of what it
        installed runs on the device's side stream (expert_cache_gather_live), so it
        overlaps whatever the current stream does next. This layer's next `refresh` settles
        the prediction: routed experts stay, the others are dropped and their copy stops;
        that `refresh`, or `join`, makes the current stream wait for the copy. Returns
        False, and does nothing, when the prediction has more ids than there are slots.

        With `along` (another layer's cache on the same device, with the same experts and
        slots), the policy step is staged instead: it runs inside the same launch as
        `along`'s next policy step, at its next `refresh`, and its copy is forked from
        there. The prediction's values are read at that launch. `along.join()`, or any
        call on this cache that reads the policy state (`refresh`, `join`, `prefetch`),
        launches a staged step on its own first."""
        ids = pred_ids if pred_ids.dtype == torch.int32 else pred_ids.to(torch.int32)
        ids = ids.contiguous()
        mk = int(ids.numel())
        if mk > self.S:
            return False
        budget = self.S if max_inserts is None else min(int(max_inserts), self.S)
        if self._riding_on is not None:  # an earlier staged step comes first
            self._riding_on._flush_rider()
        if along is None:
            self._plan()
            self._wait_copy()  # the previous copy may still read pf_miss
            cur = torch.cuda.current_stream(self.table.device)
            rc = lib().expert_cache_prefetch(ids.data_ptr(), mk, self.E, self.S, budget,
                                             *self._pf_state, cur.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"expert_cache_prefetch failed rc={rc}")
            self._copy_prefetched()
            return True
        if along is self or (along.E, along.S) != (self.E, self.S) or \
                along.table.device != self.table.device:
            raise ValueError("prefetch along= needs another layer's cache on the same device "
                             "with the same experts and slots")
        if along._rider is not None:
            along._flush_rider()
        along._rider = (self, ids, budget)
        self._riding_on = along
        return True

    def join(self) -> None:
        """Make the current stream wait for this layer's pending prefetch copy, if any.
        A prefetch staged on or with this cache is launched first, on its own."""
        if self._rider is not None:
            self._flush_rider()
        if self._riding_on is not None:
            self._riding_on._flush_rider()
        self._wait_copy()

    def _wait_copy(self) -> None:
        if self._pf_pending:
            torch.cuda.current_stream(self.table.device).wait_event(self._pf_done)
            self._pf_pending = False

    def _flush_rider(self) -> None:
        """Launch the prefetch staged on this cache on its own."""
        other, pred, budget = self._rider
        self._rider = other._riding_on = None
        other.prefetch(pred, budget)

    def _copy_prefetched(self) -> None:
        """Fork the copy of what the prefetch step just installed onto the side stream."""
        cur = torch.cuda.current_stream(self.table.device)
        side = _side_stream(self.table.device)
        if self._pf_done is None:  # two events per cache, re-recorded every prefetch
            self._pf_fork, self._pf_done = torch.cuda.Event(), torch.cuda.Event()
        self._pf_fork.record(cur)
        side.wait_event(self._pf_fork)
        # the real step that settles these installs may drop some while this copy runs: the
        # live copy stops loading those
        self._gather(self.pf_miss, self.pf_n_miss, side.cuda_stream, live=True)
        self._pf_done.record(side)
        self._pf_pending = True

    def _plan(self) -> None:
        """Resolve the gather calls against where the sources are now. vLLM's offloader
        may rebind them after the cache is built, so they are re-read every step, and the
        calls are rebuilt when one moved."""
        srcs = tuple(getattr(self.owner, n).data for n in self.names)
        key = tuple(t.data_ptr() for t in srcs)
        if key != self._gather_key:
            self._gather_calls = self._gather_plan(srcs)
            # holding the sources keeps their addresses from being reused by new tensors
            self._gather_srcs, self._gather_key = srcs, key

    def _gather(self, miss: torch.Tensor, n_miss: torch.Tensor, stream,
                live: bool = False) -> None:
        """expert_cache_gather of every mirrored tensor over one miss list, six per call,
        with the calls `_plan` resolved; with `live`, expert_cache_gather_live (a prefetch
        step's list, whose dropped predictions stop copying)."""
        h = lib()
        if live:
            fn, name = h.expert_cache_gather_live, "expert_cache_gather_live"
            tail = (miss.data_ptr(), n_miss.data_ptr(), self.slot_expert.data_ptr(),
                    self.pf_chunks, 1, stream)
        else:
            fn, name = h.expert_cache_gather, "expert_cache_gather"
            tail = (miss.data_ptr(), n_miss.data_ptr(), self.chunks, self.lanes, stream)
        for args in self._gather_calls:
            rc = fn(*args, *tail)
            if rc != 0:
                raise RuntimeError(f"{name} failed rc={rc}")

    def _gather_plan(self, srcs) -> tuple:
        """The (dst, src, bytes) x 6 argument lists of the gather calls, padded with a
        repeat (the library copies a repeated buffer once)."""
        dsts = [self.slots[n] for n in self.names]
        calls = []
        for i in range(0, len(dsts), GATHER_SLOTS):
            gd, gs = dsts[i:i + GATHER_SLOTS], list(srcs[i:i + GATHER_SLOTS])
            while len(gd) < GATHER_SLOTS:
                gd.append(gd[-1])
                gs.append(gs[-1])
            args = []
            for d, s in zip(gd, gs):
                args += [d.data_ptr(), device_address(s), _bytes_per_expert(s)]
            calls.append(tuple(args))
        return tuple(calls)
