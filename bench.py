#!/usr/bin/env python3
"""Benchmark of the per-layer expert-cache path on one MI355X.

Workload: 48 MoE layers x 128 W8A8 experts (4,732,928 B each: int8 w13 [1536, 2048], int8
w2 [2048, 768], fp32 scales [1536, 1] and [2048, 1]), ~29 GB of pinned host memory, top-8
routing at decode batch 1 (Zipf 1.1 with 0.6 per-expert repeat, one seed per layer), 64 HBM
slots per layer, LFU with decay 64, 4096-step trace. One "step" is one decode step across
all 48 layers: per layer, the fused policy step + remap kernel and the gather kernel, as the
plugin launches them, captured once into a HIP graph and replayed per step (the way vLLM
runs decode). Routing ids for the step are copied into the graph's input buffer first.

Windows of the trace (4096 steps for this workload):
  timed        steps W..W+K (--warmup W, --steps K): `value`, `ms_per_step` and `roofline`
  trace pass   the same graph replayed on to the end of the trace, steps W..4096, and then
               verified: every resident slot's bytes against the position-hash content of
               its expert (the host store holds a hash of (layer, expert, buffer, word) in
               every 4-byte word), and, in the cpu_baseline leg, every layer's per-step
               n_miss and miss list and final state against the oracle's C policy step
  steady state the second half of the trace pass (steps 2048..4096)

Printed (one JSON line on stdout; the run exits 1 if any verification fails):
  value        gathered bytes / wall time of the timed steps (GB/s), sources in host memory
  verified     the checks above, with what each covered
  trace_pass   whole-job GB/s, ms/step and hit rate over steps W..4096
  roofline     the gather kernel against the measured host->device link peak: achieved
               host->HBM GB/s over the timed steps = algorithmic bytes / what the gather
               launches add to the decode graph's time (HIP events on the launch stream,
               node substitution: decode_chain.timed); achieved_events brackets every launch
               with HIP events instead (an upper bound on its time), and
               roofline.steady_state is that over segments of the steady-state window.
               frac_trace_pass / frac_steady_state: the substitution rate over the trace
               pass and its second half; frac_*_kernel: by clock stamps inside the kernels
               (decode_chain.stamps)
  manage_remap_us_per_layer   what the fused policy+remap launch adds to the decode graph
               per layer over the trace pass: the graph's time minus that of the same graph
               with only its gathers (decode_chain), no events or profiler in the chain;
               manage_remap_kernel_us_in_chain is the kernel's own run time there (clock
               stamps), manage_remap_us_per_layer_policy_graph a graph of the policy
               launches alone, and manage_remap_us_per_layer_events the event-bracketed
               upper bound
  decode_chain the decode graph's per-node costs by substitution and by clock stamps
  hit_rate     1 - inserts / distinct routed experts over the timed steps
  hit_rate_sweep  every slot budget x LFU/LRU over the whole trace from a cold start, with
               the per-layer range
  cpu_baseline the CPU path on this machine's host: the policy restated in C (oracle/) on one
               core over the trace pass, and a CPU-driven cache (that policy deciding the
               misses, one hipMemcpyAsync per (miss, buffer)) on a sample of the timed steps
  prefetch     1,024 steps of the steady-state window with and without next-layer prefetch
               (each layer's predicted experts installed as pending by the prefetch step
               and copied on a side stream by the live gather during an earlier layer; the
               layer's real step keeps the routed ones and drops the rest), with no model
               compute and with a 50 us-per-layer compute stand-in; predictors of accuracy
               1.0 (the true routing: an upper bound) and 0.8 (each id wrong with
               probability 0.2, the wrong guess a uniformly random expert or one the layer
               routes elsewhere in the trace), one to four layers ahead, the prefetch step
               launched on its own (expert_cache_prefetch) or inside the policy launch
               (expert_cache_manage_remap_prefetch), the copy forked after the policy launch
               or after the layer's gather, or two layers' copies forked together after
               every second policy launch, and an insert budget of one
  fused        expert_cache_fused (the LRU step plus both moe_align_block_size outputs,
               block size 16) per layer-step in graph replay, 8 layers x 256 steps of three
               workloads from a cold start; cpu_baseline.fused_us_per_layer_step times the
               oracle's fused step on the same steps

    python bench.py [--steps K] [--warmup W] [--slots 64] [--policy lfu]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "vllm-expert-cache_amd"))

METRIC = ("host->HBM gather GB/s (% link peak); manage+remap µs/layer; hit rate")
WORKLOAD = "48-layer-e128"
# slot budget each workload is measured at by default, and a cap on its timed steps where
# one step moves gigabytes
TARGET_SLOTS = {"single-layer-e128": 64, "48-layer-e128": 64, "48-layer-e128-batch4": 48,
                "8-layer-e8-bf16": 4, "8-layer-e256-fp8": 128}
MAX_STEPS = {"8-layer-e256-fp8": 64}
# steps of the verified trace pass where one step moves gigabytes (default: the whole trace)
TRACE_STEPS = {"8-layer-e256-fp8": 128}
# expert_cache_fused leg: (workload, slots), and its shape
FUSED_CASES = (("48-layer-e128", 64), ("48-layer-e128-batch4", 48), ("8-layer-e256-fp8", 128))
FUSED_LAYERS, FUSED_STEPS, FUSED_BS = 8, 256, 16


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--workload", default=WORKLOAD,
                   help="48-layer-e128 (default), 48-layer-e128-batch4, 8-layer-e8-bf16, "
                        "8-layer-e256-fp8, single-layer-e128")
    p.add_argument("--steps", type=int, default=None,
                   help="timed steps (default: the rest of the workload's trace)")
    p.add_argument("--warmup", type=int, default=64)
    p.add_argument("--slots", type=int, default=None,
                   help="slot budget (default: the workload's target budget)")
    p.add_argument("--policy", choices=("lfu", "lru"), default="lfu")
    p.add_argument("--layers", type=int, default=None)
    p.add_argument("--no-trace-pass", action="store_true",
                   help="stop after the timed steps instead of replaying the rest of the "
                        "trace (the verification then covers steps 0..warmup+steps)")
    p.add_argument("--no-hit-sweep", action="store_true",
                   help="skip the per-budget, per-policy hit-rate pass over the whole trace")
    p.add_argument("--timing-segments", type=int, default=8,
                   help="segments of the timed steps re-run with per-kernel HIP events")
    p.add_argument("--segment-steps", type=int, default=8)
    p.add_argument("--cpu-steps", type=int, default=512,
                   help="timed steps in the CPU-baseline sample (0 to skip)")
    p.add_argument("--chunks", type=int, default=None)
    p.add_argument("--lanes", type=int, default=None)
    p.add_argument("--no-prefetch", action="store_true",
                   help="skip the next-layer prefetch leg")
    p.add_argument("--prefetch-compute", default="0,50",
                   help="compute stand-in per layer of the prefetch leg, us, comma-separated")
    p.add_argument("--prefetch-steps", type=int, default=1024,
                   help="steps per run of the prefetch leg (at most)")
    p.add_argument("--prefetch-from", type=int, default=None,
                   help="trace step the prefetch leg starts from (default: the steady-state "
                        "window's start; the warm-up step W gives the cold-start window)")
    p.add_argument("--prefetch-chunks", type=int, default=None,
                   help="workgroups of the prefetch leg's side copies (default: the "
                        "cache's prefetch grid)")
    p.add_argument("--no-fused", action="store_true",
                   help="skip the expert_cache_fused leg")
    p.add_argument("--no-chain", action="store_true",
                   help="skip the decode chain's per-node costs (graph substitution over the "
                        "trace pass)")
    p.add_argument("--routes", default=None,
                   help="replay a recorded trace instead of the synthetic routing: an npz "
                        "whose ids are [T, L, mk] with -1 padding (the reference's routes.npz "
                        "format); experts keep the --workload layout")
    p.add_argument("--experts", type=int, default=None,
                   help="experts per layer of a --routes trace (default: the workload's)")
    p.add_argument("--traffic-probe", action="store_true",
                   help="for rocprofv3 --pmc runs: 16 gathers of one expert each (plain, then "
                        "live), 128 policy steps of one layer, 96 decode steps of every layer "
                        "launched eagerly, and 8 plain device copies of 64 MiB (the counter "
                        "calibration), nothing else")
    return p.parse_args()


CHAIN_STEPS = 96  # decode steps of the traffic probe's eager decode loop


def traffic_probe(args):
    """Known work for the counter runs: 16 one-expert gathers, the same 16 through the live
    gather, 128 policy+remap steps of one layer back to back, the decode loop of every layer
    launched eagerly over CHAIN_STEPS steps, and 8 plain device copies whose FETCH_SIZE /
    WRITE_SIZE per byte calibrate the kernels' per-launch counters into bytes."""
    import torch

    from vllm_expert_cache import _lib, traces
    from vllm_expert_cache.cache import DEFAULT_CHUNKS, DEFAULT_LANES, device_address

    lib = _lib.lib()
    dev = torch.device("cuda:0")
    w = traces.WORKLOADS[WORKLOAD]
    E, S = w.experts, args.slots or TARGET_SLOTS[WORKLOAD]
    bufs = [b.nbytes for b in w.buffers]
    host = [torch.empty(E * b, dtype=torch.uint8, pin_memory=True) for b in bufs]
    slots = [torch.empty(S * b, dtype=torch.uint8, device=dev) for b in bufs]
    a = []
    for i in range(6):
        j = min(i, len(bufs) - 1)
        a += [ctypes.c_void_p(slots[j].data_ptr()), ctypes.c_void_p(device_address(host[j])),
              ctypes.c_long(bufs[j])]
    miss = torch.tensor([[e, e % S] for e in range(16)], dtype=torch.int32, device=dev)
    one = torch.ones(1, dtype=torch.int32, device=dev)
    s_ptr = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for r in range(16):
        rc = lib.expert_cache_gather(*a, ctypes.c_void_p(miss[r].data_ptr()),
                                     ctypes.c_void_p(one.data_ptr()), args.chunks or
                                     DEFAULT_CHUNKS, args.lanes or DEFAULT_LANES, s_ptr)
        assert rc == 0
    # the same 16 copies through the live gather, every pair live (slot_expert names it)
    slot_expert = torch.full((S,), -1, dtype=torch.int32, device=dev)
    for r in range(16):
        slot_expert.fill_(-1)
        slot_expert[r % S] = r
        rc = lib.expert_cache_gather_live(*a, ctypes.c_void_p(miss[r].data_ptr()),
                                          ctypes.c_void_p(one.data_ptr()),
                                          ctypes.c_void_p(slot_expert.data_ptr()),
                                          args.chunks or DEFAULT_CHUNKS,
                                          args.lanes or DEFAULT_LANES, s_ptr)
        assert rc == 0
    # policy+remap: 128 decode steps of the workload's layer 0 from a cold start (the
    # counters of the last 64 are the steady state)
    mk = w.mk
    ids = torch.as_tensor(traces.routing(w, 0, 128), device=dev)
    st = Layers(torch, 1, E, S, dev)
    nm = torch.zeros(1, dtype=torch.int32, device=dev)
    out = torch.zeros(mk, dtype=torch.int32, device=dev)
    for t in range(128):
        rc = lib.expert_cache_manage_remap(
            ctypes.c_void_p(ids[t].data_ptr()), 4, mk, E, S, min(E, mk), S, st.row("table", 0),
            st.row("map_cold", 0), st.row("slot_expert", 0), st.row("slot_stamp", 0),
            st.row("routed", 0), st.row("step", 0), st.row("miss", 0),
            ctypes.c_void_p(nm.data_ptr()), 1, 64, ctypes.c_void_p(out.data_ptr()), s_ptr)
        assert rc == 0
    # the decode loop, launched eagerly: every layer of the workload over CHAIN_STEPS trace
    # steps from a cold start, per layer the policy+remap step and then the gather of its
    # misses, as the decode graph orders them (every layer reads the one host store above;
    # each has its own slots). The policy counters of the last 32 steps are its in-chain
    # figures, beside the back-to-back ones of the single layer above.
    import numpy as np

    L, T = w.layers, CHAIN_STEPS
    ids = torch.as_tensor(np.stack([traces.routing(w, l, T) for l in range(L)], axis=1),
                          device=dev)
    st = Layers(torch, L, E, S, dev)
    nm = torch.zeros(L, dtype=torch.int32, device=dev)
    out = torch.zeros((L, mk), dtype=torch.int32, device=dev)
    lslots = [[torch.empty(S * b, dtype=torch.uint8, device=dev) for b in bufs]
              for _ in range(L)]
    for t in range(T):
        for l in range(L):
            rc = lib.expert_cache_manage_remap(
                ctypes.c_void_p(ids[t, l].data_ptr()), 4, mk, E, S, min(E, mk), S,
                st.row("table", l), st.row("map_cold", l), st.row("slot_expert", l),
                st.row("slot_stamp", l), st.row("routed", l), st.row("step", l),
                st.row("miss", l), ctypes.c_void_p(nm[l:].data_ptr()), 1, 64,
                ctypes.c_void_p(out[l].data_ptr()), s_ptr)
            g = []
            for i in range(6):
                j = min(i, len(bufs) - 1)
                g += [ctypes.c_void_p(lslots[l][j].data_ptr()), a[3 * j + 1], a[3 * j + 2]]
            rc |= lib.expert_cache_gather(*g, st.row("miss", l),
                                          ctypes.c_void_p(nm[l:].data_ptr()),
                                          args.chunks or DEFAULT_CHUNKS,
                                          args.lanes or DEFAULT_LANES, s_ptr)
            assert rc == 0
    n = 64 << 20
    src = torch.ones(n, dtype=torch.uint8, device=dev)
    dst = torch.empty(n, dtype=torch.uint8, device=dev)
    for _ in range(8):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"gather_launches": 16, "gather_live_launches": 16,
                      "gather_bytes_per_launch": sum(bufs),
                      "manage_remap_launches": 128, "decode_loop_layers": L,
                      "decode_loop_steps": T, "copy_launches": 8,
                      "copy_bytes_per_launch": n}), flush=True)


class Layers:
    """Device state of every layer's cache, one row per layer."""

    def __init__(self, torch, L, E, S, dev):
        i32, i64 = torch.int32, torch.int64
        self.table = torch.full((L, E), -1, dtype=i32, device=dev)
        self.map_cold = torch.arange(E, dtype=i32, device=dev).repeat(L, 1)
        self.slot_expert = torch.full((L, S), -1, dtype=i32, device=dev)
        self.slot_stamp = torch.zeros((L, S), dtype=i64, device=dev)
        self.routed = torch.zeros((L, E), dtype=torch.uint8, device=dev)
        self.step = torch.zeros((L, 1), dtype=i64, device=dev)
        self.miss = torch.zeros((L, 2 * S), dtype=i32, device=dev)
        self.n_miss = torch.zeros((L,), dtype=i32, device=dev)
        self.fields = ("table", "map_cold", "slot_expert", "slot_stamp", "routed", "step",
                       "miss")

    def row(self, name, l):
        t = getattr(self, name)
        return ctypes.c_void_p(t.data_ptr() + l * t.stride(0) * t.element_size())

    def snapshot(self):
        return {f: getattr(self, f).clone() for f in self.fields}

    def restore(self, snap):
        for f in self.fields:
            getattr(self, f).copy_(snap[f])


def main():
    args = parse()
    if args.traffic_probe:
        traffic_probe(args)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this path has no cross-GPU work (each tensor-"
              f"parallel rank runs its own identical cache); --gpus {args.gpus} is not "
              f"supported", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from vllm_expert_cache import _lib, traces
    from vllm_expert_cache.cache import (DEFAULT_CHUNKS, DEFAULT_LANES, PREFETCH_CHUNKS,
                                         device_address)

    lib = _lib.lib()  # raises if the HIP library is missing: there is no fallback
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w = traces.WORKLOADS[args.workload]
    L = args.layers or w.layers
    E, mk = w.experts, w.mk
    steps = w.steps
    name = w.name
    recorded = None
    if args.routes:
        recorded = traces.load_routes(args.routes)
        L = min(L if args.layers else recorded.shape[1], recorded.shape[1])
        recorded = recorded[:, :L]
        E = args.experts or w.experts
        if recorded.max() >= E:
            raise SystemExit(f"{args.routes}: expert id {recorded.max()} >= {E} experts; "
                             f"pass --experts")
        mk, steps = recorded.shape[2], recorded.shape[0]
        name = f"routes:{Path(args.routes).name}"
    S = args.slots or TARGET_SLOTS[w.name]
    if mk > S:
        raise SystemExit(f"{name}: {mk} routing ids per step exceed {S} slots, so every step "
                         f"reads through and there is nothing to time; pick --slots >= {mk}")
    policy = 1 if args.policy == "lfu" else 0
    decay = 64
    chunks = args.chunks or DEFAULT_CHUNKS
    lanes = args.lanes or DEFAULT_LANES
    W = min(args.warmup, steps - 1)
    K = args.steps or min(steps - W, MAX_STEPS.get(name, steps))
    T = W + K
    if T > steps:
        raise SystemExit(f"{name}: warm-up {W} + timed {K} steps exceed the trace's {steps}")
    # the trace pass replays the trace from step 0 to TP (the timed steps included) and is
    # verified at its end; TP is the whole trace unless one step moves gigabytes
    TP = T if args.no_trace_pass else max(T, min(steps, TRACE_STEPS.get(name, steps)))
    late0 = TP // 2  # the steady-state window: the second half of the trace pass
    bufs = [b.nbytes for b in w.buffers]
    B_exp = sum(bufs)

    # ---- routing, and the host expert store filled with position-hash content ------------
    t0 = time.time()
    if recorded is None:
        ids_np = np.stack([traces.routing(w, l, steps) for l in range(L)], axis=1)  # [T, L, mk]
    else:
        ids_np = np.ascontiguousarray(recorded, dtype=np.int32)
    ids_dev = torch.as_tensor(ids_np, device=dev)
    host = []  # host[l][b]: pinned [E * bytes_b]
    content = list(range(L))  # content[l]: the layer whose synthetic experts host[l] holds
    host_store = "per layer"
    try:
        for l in range(L):
            host.append([torch.empty(E * b, dtype=torch.uint8, pin_memory=True) for b in bufs])
            if l % 8 == 7:
                log(f"  pinned host store: {l + 1}/{L} layers, {time.time() - t0:.1f}s")
    except (RuntimeError, torch.AcceleratorError) as exc:
        # this host cannot pin one store per layer: every layer reads one shared store, which
        # moves the same bytes per miss from the same kind of memory
        log(f"  pinning {L * E * B_exp / 1e9:.1f} GB failed ({type(exc).__name__}); layers "
            f"share one {E * B_exp / 1e9:.1f} GB store")
        host = []
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        shared = [torch.empty(E * b, dtype=torch.uint8, pin_memory=True) for b in bufs]
        host = [shared] * L
        content = [0] * L
        host_store = f"shared by all layers (pinning {L * E * B_exp / 1e9:.1f} GB failed)"
    t1 = time.time()
    for l in sorted(set(content)):
        for b, nb in enumerate(bufs):
            traces.fill_expert_store(host[l][b], l, b, nb, E, dev)
    torch.cuda.synchronize()
    slots = [[torch.empty(S * b, dtype=torch.uint8, device=dev) for b in bufs]
             for _ in range(L)]
    log(f"setup: routing {ids_np.shape}, host store {L * E * B_exp / 1e9:.1f} GB pinned "
        f"(position-hash content written in {time.time() - t1:.1f}s), slots "
        f"{L * S * B_exp / 1e9:.1f} GB, {time.time() - t0:.1f}s")

    st = Layers(torch, L, E, S, dev)
    ids_static = torch.zeros((L, mk), dtype=torch.int32, device=dev)
    out_static = torch.zeros((L, mk), dtype=torch.int32, device=dev)
    nm_static = st.n_miss
    nm_hist = torch.zeros((TP, L), dtype=torch.int32, device=dev)
    miss_hist = torch.zeros((TP, L, 2 * S), dtype=torch.int32, device=dev)

    def row(t, l):
        return ctypes.c_void_p(t.data_ptr() + l * t.stride(0) * t.element_size())

    def gather_args(l):
        a = []
        for i in range(6):  # pad to six buffers with a repeat, as cache.refresh does
            j = min(i, len(bufs) - 1)
            a += [ctypes.c_void_p(slots[l][j].data_ptr()),
                  ctypes.c_void_p(device_address(host[l][j])), ctypes.c_long(bufs[j])]
        return a

    def manage_args(l, ids_p, nm_p, out_p):
        return (ids_p, 4, mk, E, S, min(E, mk), S, st.row("table", l), st.row("map_cold", l),
                st.row("slot_expert", l), st.row("slot_stamp", l), st.row("routed", l),
                st.row("step", l), st.row("miss", l), nm_p, policy, decay, out_p)

    M_ARGS = [manage_args(l, row(ids_static, l), row(nm_static, l), row(out_static, l))
              for l in range(L)]
    G_ARGS = [tuple(gather_args(l)) + (st.row("miss", l), row(nm_static, l), chunks, lanes)
              for l in range(L)]

    def launch_step(stream):
        s = ctypes.c_void_p(stream.cuda_stream)
        for l in range(L):
            rc = lib.expert_cache_manage_remap(*M_ARGS[l], s)
            rc |= lib.expert_cache_gather(*G_ARGS[l], s)
            if rc:
                raise RuntimeError(f"launch failed rc={rc}")

    # ---- capture one decode step into a graph --------------------------------------------
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    snap0 = st.snapshot()
    with torch.cuda.stream(side):
        launch_step(side)  # warm-up launch outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    st.restore(snap0)
    nm_static.zero_()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch_step(torch.cuda.current_stream())
    torch.cuda.synchronize()

    def run_steps(t_from, t_to, snaps):
        for t in range(t_from, t_to):
            if t in snaps:
                for f in st.fields:
                    snaps[t][f].copy_(getattr(st, f), non_blocking=True)
            ids_static.copy_(ids_dev[t], non_blocking=True)
            graph.replay()
            nm_hist[t].copy_(nm_static, non_blocking=True)
            miss_hist[t].copy_(st.miss, non_blocking=True)

    # ---- warm-up, the timed steps, then the rest of the trace pass ------------------------
    # state snapshots at the starts of the segments re-run with per-kernel events: the timed
    # window's, and the steady-state window's (second half of the trace pass)
    nseg = max(1, min(args.timing_segments, K))
    seg_len = max(1, min(args.segment_steps, K // nseg))
    seg_starts = _spread(W, T, nseg, seg_len)
    late_len = min(args.segment_steps, max(1, (TP - late0) // max(1, args.timing_segments)))
    late_starts = _spread(late0, TP, args.timing_segments, late_len) if TP - late0 >= 16 \
        else []
    pf0 = late0 if late_starts else W  # the prefetch leg starts from a steady state too
    if args.prefetch_from is not None:
        pf0 = min(max(args.prefetch_from, 0), TP - 1)
    snaps = {t: st.snapshot() for t in set(seg_starts) | set(late_starts) | {W, pf0}}
    run_steps(0, W, snaps)
    torch.cuda.synchronize()
    ev_a, ev_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    ev_a.record()
    run_steps(W, T, snaps)
    ev_b.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    elapsed_s = max(wall, ev_a.elapsed_time(ev_b) / 1e3)
    rest_s = 0.0
    if TP > T:
        wall0 = time.perf_counter()
        ev_a.record()
        run_steps(T, TP, snaps)
        ev_b.record()
        torch.cuda.synchronize()
        rest_s = max(time.perf_counter() - wall0, ev_a.elapsed_time(ev_b) / 1e3)
    nm = nm_hist.cpu().numpy()
    inserts = int(nm[W:T].sum())
    distinct = int(_distinct(np, ids_np[W:T]).sum())
    gathered = inserts * B_exp
    value = gathered / elapsed_s / 1e9
    log(f"timed: {K} steps (trace steps {W}..{T}) in {elapsed_s:.2f}s "
        f"({1e3 * elapsed_s / K:.3f} ms/step), {inserts} inserts, {gathered / 1e9:.1f} GB -> "
        f"{value:.2f} GB/s")
    pass_inserts = int(nm[W:TP].sum())
    pass_s = elapsed_s + rest_s
    trace_pass = {
        "trace_steps": [W, TP], "ms_per_step": round(1e3 * pass_s / (TP - W), 4),
        "GBps": round(pass_inserts * B_exp / pass_s / 1e9, 3), "inserts": pass_inserts,
        "hit_rate": round(1.0 - pass_inserts / int(_distinct(np, ids_np[W:TP]).sum()), 5),
        "hit_rate_from_cold_start": round(
            1.0 - int(nm[:TP].sum()) / int(_distinct(np, ids_np[:TP]).sum()), 5),
        "def": "the same graph replayed from step W to the end of the trace pass (the timed "
               "steps included): whole-job GB/s and hit rate over those steps"}
    log(f"trace pass: steps {W}..{TP} at {trace_pass['ms_per_step']} ms/step, "
        f"{trace_pass['GBps']} GB/s, hit rate {trace_pass['hit_rate']}")

    # ---- verification of the trace pass's slot bytes (its state is checked against the ----
    # ---- oracle in the cpu_baseline leg) -------------------------------------------------
    final = st.snapshot()
    t1 = time.time()
    slot_ok, resident = True, 0
    for l in range(L):
        for b, nb in enumerate(bufs):
            ok, n = traces.slots_match(slots[l][b], st.slot_expert[l], content[l], b, nb)
            slot_ok = slot_ok and ok
        resident += n
    log(f"verify: {resident} resident slots x {B_exp} B against the position hash: "
        f"{'equal' if slot_ok else 'MISMATCH'} ({time.time() - t1:.1f}s)")
    verified = {"slot_bytes": slot_ok, "resident_slots": resident,
                "slot_bytes_checked": resident * B_exp, "layers": L, "trace_steps": [0, TP],
                "state": None, "n_miss_per_step": None, "miss_lists_per_step": None,
                "def": "after the trace pass: every resident slot's bytes against the "
                       "position-hash content of the expert its slot_expert names; every "
                       "layer's per-step n_miss and miss list and final state (table, "
                       "map_cold, slot_expert, slot_stamp, step) against the oracle's policy "
                       "step in C from the same cold start (cpu_baseline leg)"}

    # ---- per-kernel durations: segments re-run from their snapshots, HIP events around ----
    # ---- every launch on the launch stream ----------------------------------------------
    stream = torch.cuda.current_stream()
    s_ptr = ctypes.c_void_p(stream.cuda_stream)

    def event_segments(starts, n):
        ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
                torch.cuda.Event(enable_timing=True)) for _ in range(L)] for _ in range(n)]
        seg_out = torch.zeros((n, L, mk), dtype=torch.int32, device=dev)
        seg_nm = torch.zeros((n, L), dtype=torch.int32, device=dev)
        man, gat, wn = [], [], []
        for t0s in starts:
            st.restore(snaps[t0s])
            torch.cuda.synchronize()
            torch.cuda._sleep(int(2e8))  # hold the stream while the segment is queued
            for i in range(n):
                t = t0s + i
                for l in range(L):
                    e0, e1, e2 = ev[i][l]
                    e0.record(stream)
                    rc = lib.expert_cache_manage_remap(
                        *manage_args(l, row(ids_dev[t], l), row(nm_static, l),
                                     row(seg_out[i], l)), s_ptr)
                    e1.record(stream)
                    rc |= lib.expert_cache_gather(*G_ARGS[l], s_ptr)
                    e2.record(stream)
                    if rc:
                        raise RuntimeError(f"launch failed rc={rc}")
                seg_nm[i].copy_(nm_static)  # outside the event brackets
            torch.cuda.synchronize()
            man.append([[ev[i][l][0].elapsed_time(ev[i][l][1]) * 1e3 for l in range(L)]
                        for i in range(n)])
            gat.append([[ev[i][l][1].elapsed_time(ev[i][l][2]) * 1e3 for l in range(L)]
                        for i in range(n)])
            got = seg_nm.cpu().numpy()
            assert np.array_equal(got, nm[t0s:t0s + n]), "segment diverged from the trace pass"
            wn.append(got)
        man, gat, wn = np.array(man), np.array(gat), np.array(wn)
        with_miss = wn > 0
        fig = {"achieved": wn.sum() * B_exp / (gat.sum() * 1e-6) / 1e9,
               "with_miss": (wn[with_miss].sum() * B_exp / (gat[with_miss].sum() * 1e-6) / 1e9
                             if with_miss.any() else None),
               "zero_us": float(gat[~with_miss].mean()) if (~with_miss).any() else None,
               "gather_us": float(gat.mean()), "manage_us": float(man.mean()),
               "manage_p50": float(np.median(man)), "launches": int(wn.size),
               "launches_with_miss": int(with_miss.sum()), "inserts": int(wn.sum())}
        log(f"{len(starts)} segments x {n} steps from {starts[0]}: manage+remap "
            f"{fig['manage_us']:.2f} us/layer (p50 {fig['manage_p50']:.2f}), gather "
            f"{fig['gather_us']:.1f} us/launch, {fig['achieved']:.2f} GB/s over all launches, "
            f"{fig['with_miss']} GB/s over launches with a miss, {fig['zero_us']} us for a "
            f"launch with no miss")
        return fig

    tw = event_segments(seg_starts, seg_len)
    late = event_segments(late_starts, late_len) if late_starts else None
    st.restore(final)

    # ---- host->device link peak -------------------------------------------------------------
    peak, peak_detail = link_peak(torch, lib, s_ptr, dev)

    # ---- latency floor: an empty kernel node in a graph of L, replays behind a hold --------
    hold = Hold(torch)
    ge = torch.cuda.CUDAGraph()
    with torch.cuda.graph(ge):
        for _ in range(L):
            torch.cuda._sleep(0)
    ge.replay()
    torch.cuda.synchronize()
    empty_s = sum(s for _, _, s in hold.time(0, 256, lambda t: ge.replay()))
    empty_us = empty_s * 1e6 / (256 * L)
    del ge
    log(f"empty kernel node in a graph of {L}: {empty_us:.2f} us")

    # ---- the decode chain's per-node costs, by substitution --------------------------------
    chain = None if args.no_chain else chain_costs(
        torch, lib, hold, graph, M_ARGS, gather_args, st, snaps[W], final, ids_dev,
        ids_static, nm_hist, miss_hist, nm[:TP], W, T, TP, late0, L, S, B_exp, chunks, lanes,
        peak, dev)
    verified["chain_rerun_state"] = None if chain is None else chain.pop("rerun_state_equal")
    stamps = None if args.no_chain else chain_stamps(
        torch, np, hold, M_ARGS, G_ARGS, st, snaps[W], final, ids_dev, ids_static, nm[:TP], W,
        TP, late0, L, B_exp, chunks * lanes, peak, dev)
    verified["stamped_rerun_state"] = None if stamps is None else \
        stamps.pop("rerun_state_equal")
    if chain is not None:
        chain["stamps"] = stamps

    # ---- CPU baseline: C policy on one core + hipMemcpyAsync per (miss, buffer); the same --
    # ---- C policy over the trace pass checks the GPU's states ----------------------------
    check, policy_timing = oracle_check(np, ids_np, L, E, S, policy, decay, TP, nm[:TP],
                                        miss_hist.cpu().numpy(), final)
    verified.update(check)
    cpu = None
    if args.cpu_steps > 0:
        cpu = cpu_baseline(args, torch, np, ids_np, host, slots, bufs, snaps[W], L, E, S, mk,
                           policy, decay, W, policy_timing)

    prefetch = None
    if not args.no_prefetch:
        # about 130 GB moved per run at most: 1,024 steps of the default workload, fewer
        # where experts are hundreds of MB
        per_step = max(1.0, pass_inserts * B_exp / (TP - W))
        pw = max(32, min(args.prefetch_steps, int(130e9 / per_step)))
        prefetch = prefetch_leg(torch, np, lib, ids_np, ids_dev, G_ARGS, snaps[pf0], L, E, S,
                                mk, policy, decay, pf0, min(steps, pf0 + pw), B_exp, chunks,
                                lanes, dev, peak, slots, content, bufs, window=pw,
                                pf_chunks=args.prefetch_chunks or PREFETCH_CHUNKS,
                                compute=tuple(float(c) for c in
                                              args.prefetch_compute.split(",")))
    verified["prefetch"] = None if prefetch is None else prefetch["verified"]["all"]

    fused = None if args.no_fused else fused_leg(torch, np, lib, dev, hold)

    sweep = None
    if not args.no_hit_sweep:
        sweep = hit_rate_sweep(torch, np, lib, w, ids_np, ids_dev, L, E, mk, decay, dev, hold)
    if chain is not None:
        manage_us = chain["trace_pass"]["manage_remap_us_per_layer"]
        manage_def = chain["manage_remap_def"]
    else:
        manage_us = round(tw["manage_us"], 3)
        manage_def = "HIP events around each launch (adds the launch's dispatch): an upper bound"
    policy_graph_us = next((x["graph_us_per_layer"] for x in sweep or []
                            if x.get("slots") == S and x.get("policy") == args.policy), None)
    verified["all"] = all(verified[k] is True for k in
                          ("slot_bytes", "state", "n_miss_per_step", "miss_lists_per_step")) \
        and all(verified[k] is not False for k in ("chain_rerun_state", "stamped_rerun_state",
                                                   "prefetch"))

    traffic = _traffic()
    if chain is not None:
        achieved = chain["timed"]["gather_GBps"]
        achieved_how = ("gathered bytes / what the gather launches add to the decode graph's "
                        "time (HIP events on the launch stream around replays of the graph "
                        "and of the same graph without its gathers, each from the same "
                        "snapshot behind a stream hold; decode_chain.timed)")
    else:
        achieved = tw["achieved"]
        achieved_how = ("gathered bytes / summed gather launch time, HIP events around each "
                        "launch (achieved_events)")

    def rounded(v, n=3):
        return None if v is None else round(v, n)

    res = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(1e3 * elapsed_s / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic" if recorded is None else "recorded routing, synthetic experts",
        "config": {"workload": name, "expert_layout": w.name, "layers": L, "experts": E,
                   "ids_per_step": mk, "top_k": None if recorded is not None else w.top_k,
                   "tokens_per_step": None if recorded is not None else w.tokens,
                   "slots": S, "policy": args.policy,
                   "decay": decay, "bytes_per_expert": B_exp, "host_store_GB":
                   round(L * E * B_exp / 1e9, 2), "host_store": host_store,
                   "expert_content": "position hash of (layer, expert, buffer, word)",
                   "gather_grid": [chunks, lanes],
                   "timed_trace_steps": [W, T], "trace_steps": steps},
        "verified": verified,
        "hit_rate": round(1.0 - inserts / distinct, 5),
        "inserts": inserts,
        "trace_pass": trace_pass,
        "manage_remap_us_per_layer": manage_us,
        "manage_remap_def": manage_def,
        "manage_remap_us_per_layer_steady_state":
            None if chain is None else chain["steady_state"]["manage_remap_us_per_layer"],
        "manage_remap_substitution_noise_us":
            None if chain is None else chain["trace_pass"]["noise_us_per_layer"],
        "manage_remap_over_empty_node_us":
            None if chain is None else chain["trace_pass"]["manage_remap_over_empty_node_us"],
        "empty_node_in_chain_us":
            None if chain is None else chain["trace_pass"]["empty_node_us"],
        "manage_remap_kernel_us_in_chain":
            None if stamps is None else stamps["chain"]["trace_pass"]["policy_us"]["mean"],
        "manage_remap_us_per_layer_policy_graph": policy_graph_us,
        "manage_remap_us_per_layer_events": round(tw["manage_us"], 3),
        "empty_kernel_graph_us": round(empty_us, 3),
        "decode_chain": chain,
        "manage_remap_counters": _manage_counters(),
        "gather_us_per_launch": round(tw["gather_us"], 3),
        "gather_GBps_launches_with_miss": rounded(tw["with_miss"]),
        "gather_us_launch_without_miss": rounded(tw["zero_us"]),
        "link_peak": peak_detail,
        "roofline": {"bound": "host-link", "kernel": "gather_k",
                     "achieved": round(achieved, 3),
                     "peak": round(peak, 3), "unit": "GB/s",
                     "frac": round(achieved / peak, 4),
                     "achieved_events": round(tw["achieved"], 3),
                     "frac_events": round(tw["achieved"] / peak, 4),
                     # the metric's other two parts, as scalars beside the gather's
                     "policy_kernel": "manage_k (policy step + fused remap, one wavefront)",
                     "policy_bound": "latency",
                     "policy_us_per_layer": manage_us,
                     "policy_kernel_us_in_chain":
                         None if stamps is None
                         else stamps["chain"]["trace_pass"]["policy_us"]["mean"],
                     "policy_empty_node_us":
                         None if chain is None else chain["trace_pass"]["empty_node_us"],
                     "policy_target_us": 10.0,
                     "policy_def": "us/layer the launch adds to the decode graph (node "
                                   "substitution); kernel: clock stamps; empty node: same "
                                   "place",
                     "hit_rate_trace_pass": trace_pass["hit_rate"],
                     "frac_trace_pass": None if chain is None
                     else chain["trace_pass"]["gather_frac"],
                     "frac_steady_state": None if chain is None
                     else chain["steady_state"]["gather_frac"],
                     "frac_trace_pass_kernel": None if stamps is None
                     else stamps["chain"]["trace_pass"]["gather_kernel_frac"],
                     "frac_steady_state_kernel": None if stamps is None
                     else stamps["chain"]["steady_state"]["gather_kernel_frac"],
                     "frac_trace_pass_whole_job": round(trace_pass["GBps"] / peak, 4),
                     "inserts_per_launch_steady": round(float(nm[late0:TP].sum()) /
                                                        max(1, (TP - late0) * L), 4),
                     "achieved_launches_with_miss": rounded(tw["with_miss"]),
                     "frac_launches_with_miss": None if tw["with_miss"] is None
                     else round(tw["with_miss"] / peak, 4),
                     "traffic": None if traffic is None else traffic["bytes_per_launch"],
                     "traffic_detail": traffic,
                     "achieved_def": f"{achieved_how} in the timed window (trace steps "
                                     f"{W}..{T}{', a cold start' if W < 64 else ''}). "
                                     f"achieved_events: gathered bytes / summed gather "
                                     f"launch time over all launches of the same window, "
                                     f"launches without a miss included: {nseg} segments x "
                                     f"{seg_len} steps x {L} layers re-run from snapshots, "
                                     f"HIP events around each launch (which add the launch's "
                                     f"dispatch); achieved_launches_with_miss counts only "
                                     f"launches that copy, gather_us_launch_without_miss is "
                                     f"the rest's cost; steady_state is the same over the "
                                     f"second half of the trace pass. frac_trace_pass and "
                                     f"frac_steady_state: "
                                     f"gathered bytes / what the gather nodes add to the "
                                     f"decode graph (its time minus the time of the same "
                                     f"graph without them) over trace steps {W}..{TP} and "
                                     f"{late0}..{TP}, no events or profiler in the chain "
                                     f"(decode_chain); frac_trace_pass_kernel and "
                                     f"frac_steady_state_kernel: gathered bytes / the gather "
                                     f"kernels' own durations in the same windows, from clock "
                                     f"stamps inside stamped copies of the kernels "
                                     f"(decode_chain.stamps); frac_trace_pass_whole_job: "
                                     f"trace_pass.GBps, the whole step's wall time",
                     "peak_def": "measured: the best single repetition of hipMemcpyAsync H2D "
                                 "of 2 GiB pinned and of the gather kernel on one 2 GiB slab "
                                 "(16, 32 and 64 workgroups), 3 repetitions each (link_peak)",
                     "steady_state": None if late is None else {
                         "trace_steps": [late0, TP], "trace_inserts": int(nm[late0:TP].sum()),
                         "segments": len(late_starts),
                         "segment_steps": late_len, "achieved": round(late["achieved"], 3),
                         "frac": round(late["achieved"] / peak, 4),
                         "achieved_launches_with_miss": rounded(late["with_miss"]),
                         "frac_launches_with_miss": None if late["with_miss"] is None
                         else round(late["with_miss"] / peak, 4),
                         "gather_us_launch_without_miss": rounded(late["zero_us"]),
                         "inserts_per_launch": round(late["inserts"] / late["launches"], 4),
                         "manage_remap_us_per_layer_events": round(late["manage_us"], 3)}},
        "cpu_baseline": cpu,
        "prefetch": prefetch,
        "fused": fused,
        "hit_rate_sweep": sweep,
    }
    print(json.dumps(res), flush=True)
    if not verified["all"]:
        log(f"VERIFICATION FAILED: {verified}")
        sys.exit(1)


def chunk_points(lo, hi, chunk, cuts=()):
    """Boundaries of the timed chunks of steps [lo, hi): every multiple of `chunk` inside,
    each cut inside, and both ends; sorted."""
    return sorted({lo, hi} | {c for c in cuts if lo < c < hi} |
                  set(range((lo // chunk + 1) * chunk, hi, chunk)))


class Hold:
    """Times short GPU work with stream holds: each chunk of steps is queued behind a spin
    kernel on the current stream, so the GPU runs the chunk back to back instead of at the
    rate the host queues it. The hold is sized from the host's queueing time of the previous
    chunk; a chunk that took the host longer to queue than its hold is counted in `late`
    (the GPU may have waited for the host there)."""

    def __init__(self, torch, first_us=20000.0, min_us=1000.0):
        self.torch = torch
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        torch.cuda._sleep(int(2e6))
        b.record()
        torch.cuda.synchronize()
        self.cyc_per_us = 2e6 / (a.elapsed_time(b) * 1e3)
        self.hold_us, self.first_us, self.min_us = first_us, first_us, min_us
        self.chunks = self.late = 0

    def time(self, lo, hi, enqueue, chunk=16, cuts=()):
        """Runs enqueue(t) for t in [lo, hi) in chunks that end at multiples of `chunk` and
        at each of `cuts`; returns [(c0, c1, GPU seconds of chunk [c0, c1))]."""
        torch = self.torch
        pts = chunk_points(lo, hi, chunk, cuts)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        out = []
        self.hold_us = self.first_us
        for c0, c1 in zip(pts[:-1], pts[1:]):
            torch.cuda.synchronize()
            torch.cuda._sleep(int(self.hold_us * self.cyc_per_us))
            a.record()
            h0 = time.perf_counter()
            for t in range(c0, c1):
                enqueue(t)
            host_us = (time.perf_counter() - h0) * 1e6
            b.record()
            torch.cuda.synchronize()
            out.append((c0, c1, a.elapsed_time(b) * 1e-3))
            self.chunks += 1
            self.late += host_us > self.hold_us
            self.hold_us = max(self.min_us, 2.0 * host_us)
        return out

    def record(self):
        return {"chunks": self.chunks, "late_chunks": self.late,
                "spin_cycles_per_us": round(self.cyc_per_us, 1)}


def substitution_window(times, lo, hi, nm, L, B_exp, peak):
    """The decode chain's per-node costs over trace steps [lo, hi) from the substitution
    variants' timed chunks: times[variant] = [(c0, c1, GPU seconds of chunk [c0, c1))], with
    variants full, gathers, gathers_again, empty+gather and policy (chain_costs); only the
    chunks that lie inside the window count. nm[t, l] is the inserts of step t, layer l."""
    n = hi - lo
    t = {k: sum(s for c0, c1, s in v if c0 >= lo and c1 <= hi) for k, v in times.items()}
    per = 1e6 / (n * L)
    moved = float(nm[lo:hi].sum()) * B_exp
    gather_s = t["full"] - t["policy"]
    return {"trace_steps": [lo, hi],
            "ms_per_step": round(1e3 * t["full"] / n, 4),
            "manage_remap_us_per_layer": round((t["full"] - t["gathers"]) * per, 3),
            "noise_us_per_layer": round(abs(t["gathers_again"] - t["gathers"]) * per, 3),
            "empty_node_us": round((t["empty+gather"] - t["gathers"]) * per, 3),
            "manage_remap_over_empty_node_us": round((t["full"] - t["empty+gather"]) * per, 3),
            "policy_graph_us_per_layer": round(t["policy"] * per, 3),
            "gather_us_per_launch": round(gather_s * per, 3),
            "gather_GBps": round(moved / gather_s / 1e9, 3),
            "gather_frac": round(moved / gather_s / 1e9 / peak, 4),
            "inserts": int(nm[lo:hi].sum()),
            "seconds": {k: round(v, 5) for k, v in t.items()}}


def chain_costs(torch, lib, hold, graph, m_args, gather_args, st, snap, final, ids_dev,
                ids_static, nm_hist, miss_hist, nm, W, T, TP, late0, L, S, B_exp, chunks,
                lanes, peak, dev):
    """What each node of the decode graph costs inside the chain, measured by substitution:
    the graph's step time against the same step with some of its nodes taken out or
    replaced, each replayed over the same trace steps behind stream holds. No events sit
    between the nodes and no profiler is attached, so every figure is the chain's own.

      full         the decode graph: per layer the policy+remap launch, then the gather
      gathers      per layer only the gather, of the miss list the full graph recorded at
                   that step and layer (copied in per step, so the same bytes move)
      empty+gather per layer an empty kernel node in place of the policy launch, then the
                   same gather
      policy       per layer only the policy+remap launch
    The gathers-only variant is replayed a second time; the two replays' difference per
    layer-step (noise_us_per_layer) is the scale below which a difference means nothing.

    Every variant copies the step's routing ids and recorded miss lists into its inputs
    before the replay, so the per-step copies cancel in the differences:
      policy+remap per layer = (full - gathers) / (steps x L)
      empty node per layer   = (empty+gather - gathers) / (steps x L)
      gather per launch      = (full - policy) / (steps x L), and the gather's in-chain rate
                               is the gathered bytes over (full - policy).
    Each variant is timed per window: the timed steps W..T, the trace pass W..TP and its
    second half late0..TP. The policy and full variants restart from the snapshot at step
    W; the full variant's final state must equal the trace pass's (rerun_state_equal)."""
    i32 = torch.int32
    # recorded miss lists as gather inputs: row l = [n_miss, e0, s0, e1, s1, ...]
    rec_dev = torch.cat([nm_hist[:TP, :, None], miss_hist[:TP]], dim=2).contiguous()
    rec_static = torch.zeros((L, 1 + 2 * S), dtype=i32, device=dev)
    rs = rec_static.stride(0) * rec_static.element_size()
    rec_args = [tuple(gather_args(l)) + (ctypes.c_void_p(rec_static.data_ptr() + l * rs + 4),
                                         ctypes.c_void_p(rec_static.data_ptr() + l * rs),
                                         chunks, lanes) for l in range(L)]

    def capture(launch):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            launch(s)
        torch.cuda.synchronize()
        return g

    def gathers(s, empty=False):
        for l in range(L):
            if empty:
                torch.cuda._sleep(0)
            if lib.expert_cache_gather(*rec_args[l], s):
                raise RuntimeError("gather launch failed")

    def policy(s):
        for l in range(L):
            if lib.expert_cache_manage_remap(*m_args[l], s):
                raise RuntimeError("policy launch failed")

    g_only = capture(gathers)
    # the gathers-only variant runs twice: the two runs' difference is the substitution's
    # noise (the host link's rate varies a little from pass to pass)
    variants = {"gathers": g_only, "empty+gather": capture(lambda s: gathers(s, empty=True)),
                "policy": capture(policy), "full": graph, "gathers_again": g_only}
    times = {}
    for name, g in variants.items():
        def enqueue(t, g=g):
            ids_static.copy_(ids_dev[t], non_blocking=True)
            rec_static.copy_(rec_dev[t], non_blocking=True)
            g.replay()

        if name in ("policy", "full"):
            st.restore(snap)
        times[name] = hold.time(W, TP, enqueue, cuts=(late0, T))
        log(f"decode chain, {name}: {sum(x[2] for x in times[name]):.4f} s over steps "
            f"{W}..{TP}")
    rerun_equal = all(torch.equal(getattr(st, f), final[f]) for f in st.fields)
    del g_only
    for name in ("gathers", "empty+gather", "policy", "gathers_again"):
        del variants[name]

    def window(lo, hi=TP):
        return substitution_window(times, lo, hi, nm, L, B_exp, peak)

    out = {"timed": window(W, T), "trace_pass": window(W), "steady_state": window(late0),
           "hold": hold.record(), "rerun_state_equal": rerun_equal,
           "manage_remap_def": f"what the policy+remap launch adds to the decode graph per "
                               f"layer, over trace steps {W}..{TP}: the graph's time minus "
                               f"that of the same graph with only its gathers (fed the "
                               f"recorded miss lists), per layer-step; no events or "
                               f"profiler in the chain (decode_chain)",
           "def": chain_costs.__doc__.split("\n\n")[1].strip()}
    tp, ss, tm = out["trace_pass"], out["steady_state"], out["timed"]
    log(f"decode chain over the timed steps {W}..{T}: gather {tm['gather_GBps']} GB/s "
        f"({tm['gather_frac']}), {tm['gather_us_per_launch']} us per launch, policy+remap "
        f"{tm['manage_remap_us_per_layer']} us/layer")
    log(f"decode chain over steps {W}..{TP}: policy+remap {tp['manage_remap_us_per_layer']} "
        f"us/layer (noise {tp['noise_us_per_layer']}, empty node {tp['empty_node_us']}, "
        f"policy-only graph "
        f"{tp['policy_graph_us_per_layer']}), gather {tp['gather_GBps']} GB/s "
        f"({tp['gather_frac']}); steady state from {late0}: policy+remap "
        f"{ss['manage_remap_us_per_layer']} us/layer, gather {ss['gather_GBps']} GB/s "
        f"({ss['gather_frac']}); re-run state {'equal' if rerun_equal else 'MISMATCH'}")
    return out


def _stamps_lib():
    """bench_stamps.so (bench_stamps.hip, built by __graft_entry__.build()), bound."""
    from vllm_expert_cache._lib import SIGNATURES

    path = ROOT / "bench_stamps.so"
    if not path.is_file():
        raise FileNotFoundError(f"{path} missing: run __graft_entry__.build()")
    h = ctypes.CDLL(str(path))
    P = ctypes.c_void_p
    for name, base in (("stamped_manage_remap", "expert_cache_manage_remap"),
                       ("stamped_gather", "expert_cache_gather")):
        f = getattr(h, name)
        f.restype = ctypes.c_int
        f.argtypes = SIGNATURES[base][:-1] + [P, P]  # ... row(s), stream
    h.stamped_empty.restype = ctypes.c_int
    h.stamped_empty.argtypes = [P, P]
    h.stamped_clock_khz.restype = ctypes.c_int
    h.stamped_clock_khz.argtypes = [ctypes.c_int]
    return h


def chain_stamps(torch, np, hold, m_args, g_args, st, snap, final, ids_dev, ids_static, nm,
                 W, TP, late0, L, B_exp, grid, peak, dev):
    """The decode chain's kernel times from inside the kernels: the decode graph rebuilt
    with bench_stamps.so's stamped copies of the policy+remap and gather kernels (the
    product's device code between two reads of the GPU's constant-rate clock) and replayed
    over trace steps W..TP from the snapshot at W, the stamps of every launch kept. Then the
    same with the policy launches alone (back to back). Per window (the trace pass, and the
    steady state from late0):
      policy_us        the policy+remap kernel, first instruction to its stores completed
      into_policy_us   the previous layer's gather ending (its last workgroup) to the policy
                       kernel's first instruction: what the chain takes to start it
      into_gather_us   the policy kernel's end to the gather's first workgroup starting
      gather_us        the gather's first workgroup starting to its last one ending, for
                       launches without a miss and with one
      gather_kernel_GBps  gathered bytes / summed gather durations: the kernel-only rate
    The first layer of each step is left out of the gap figures (the per-step copies sit
    before it). The stamped run's final state must equal the trace pass's."""
    sl = _stamps_lib()
    rows = torch.zeros((L, 1 + grid, 2), dtype=torch.int64, device=dev)
    n = TP - W
    hist = torch.zeros((n, L, 1 + grid, 2), dtype=torch.int64, device=dev)

    def rp(l, k):
        return ctypes.c_void_p(rows.data_ptr() + (l * (1 + grid) + k) * 16)

    # the clock's rate: two stamped empty kernels around a 200 ms spin, timed by HIP events
    # and by the host's clock (which the stamps are converted with: the host's launch and
    # synchronisation add ~0.01 %), beside the rate the device reports
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0 = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # a first launch loads the library's code object (milliseconds on the host), which must
    # not fall inside the interval
    assert sl.stamped_empty(rp(0, 0), s0) == 0
    torch.cuda.synchronize()
    h0 = time.perf_counter()
    a.record()
    assert sl.stamped_empty(rp(0, 0), s0) == 0
    torch.cuda._sleep(int(200000 * hold.cyc_per_us))
    assert sl.stamped_empty(rp(1, 0), s0) == 0
    b.record()
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - h0
    r = rows.cpu().numpy()
    ticks = float(r[1, 0, 0] - r[0, 0, 0])
    mhz = ticks / (wall_s * 1e6)
    clock = {"MHz": round(mhz, 3), "MHz_by_events": round(ticks / (a.elapsed_time(b) * 1e3), 3),
             "MHz_reported": sl.stamped_clock_khz(0) / 1e3,
             "events_over_wall": round(a.elapsed_time(b) * 1e-3 / wall_s, 5),
             "def": "stamp ticks between two stamped kernels around a 200 ms spin, over the "
                    "host's wall time of the interval (MHz, used to convert the stamps) and "
                    "over HIP events' elapsed time (MHz_by_events); MHz_reported is the "
                    "device's hipDeviceAttributeWallClockRate"}

    def capture(policy_only):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for l in range(L):
                rc = sl.stamped_manage_remap(*m_args[l], rp(l, 0), s)
                if not policy_only:
                    rc |= sl.stamped_gather(*g_args[l], rp(l, 1), s)
                if rc:
                    raise RuntimeError(f"stamped launch failed rc={rc}")
        torch.cuda.synchronize()
        return g

    out = {"clock_MHz": round(float(mhz), 3), "clock": clock}
    for name in ("chain", "policy_only"):
        g = capture(name == "policy_only")
        st.restore(snap)
        rows.zero_()

        def enqueue(t):
            ids_static.copy_(ids_dev[t], non_blocking=True)
            g.replay()
            hist[t - W].copy_(rows, non_blocking=True)

        hold.time(W, TP, enqueue)
        del g
        if name == "chain":
            out["rerun_state_equal"] = all(torch.equal(getattr(st, f), final[f])
                                           for f in st.fields)
        h = hist.cpu().numpy().astype(np.float64) / mhz  # us
        out[name] = {}
        for wname, lo in (("trace_pass", W), ("steady_state", late0)):
            x = h[lo - W:]
            pol = x[:, :, 0, 1] - x[:, :, 0, 0]
            fig = {"trace_steps": [lo, TP], "policy_us": _stats(np, pol)}
            if name == "chain":
                g0, g1 = x[:, :, 1:, 0].min(-1), x[:, :, 1:, 1].max(-1)
                gat = g1 - g0
                moved = nm[lo:TP] > 0
                fig["into_policy_us"] = _stats(np, x[:, 1:, 0, 0] - g1[:, :-1])
                fig["into_gather_us"] = _stats(np, g0[:, 1:] - x[:, 1:, 0, 1])
                fig["gather_us_without_miss"] = _stats(np, gat[~moved])
                fig["gather_us_with_miss"] = _stats(np, gat[moved])
                nbytes = float(nm[lo:TP].sum()) * B_exp
                fig["gather_kernel_GBps"] = round(nbytes / (gat.sum() * 1e-6) / 1e9, 3)
                fig["gather_kernel_frac"] = round(fig["gather_kernel_GBps"] / peak, 4)
                fig["gather_kernel_GBps_launches_with_miss"] = round(
                    nbytes / (gat[moved].sum() * 1e-6) / 1e9, 3) if moved.any() else None
                fig["layer_us"] = round(float((x[:, 1:, 1:, 1].max(-1) -
                                               g1[:, :-1]).mean()), 3)
            else:
                fig["into_policy_us"] = _stats(np, x[:, 1:, 0, 0] - x[:, :-1, 0, 1])
            out[name][wname] = fig
    c, p = out["chain"]["trace_pass"], out["policy_only"]["trace_pass"]
    log(f"stamps (clock {mhz:.1f} MHz), trace pass: policy+remap kernel "
        f"{c['policy_us']['mean']} us in the chain (p50 {c['policy_us']['p50']}), "
        f"{p['policy_us']['mean']} us back to back; into policy {c['into_policy_us']['mean']}, "
        f"into gather {c['into_gather_us']['mean']} us; gather kernel-only "
        f"{c['gather_kernel_GBps']} GB/s ({c['gather_kernel_frac']}); steady state "
        f"{out['chain']['steady_state']['gather_kernel_GBps']} GB/s")
    out["def"] = " ".join(chain_stamps.__doc__.split("\n\n")[0].split())
    return out


def _stats(np, x):
    x = np.asarray(x, dtype=np.float64).ravel()
    if x.size == 0:
        return None
    return {"mean": round(float(x.mean()), 3), "p10": round(float(np.percentile(x, 10)), 3),
            "p50": round(float(np.median(x)), 3), "p90": round(float(np.percentile(x, 90)), 3),
            "n": int(x.size)}


def link_peak(torch, lib, s_ptr, dev, n_bytes=2 << 30, reps=3, grids=(16, 32, 64)):
    """The host->device link's peak, measured: hipMemcpyAsync H2D of n_bytes from pinned
    memory, and the gather kernel copying one n_bytes slab on grids of 16, 32 and 64
    workgroups; each `reps` times after a warm-up, HIP events around each. The peak is the
    best single repetition of any method."""
    from vllm_expert_cache.cache import device_address

    src = torch.empty(n_bytes, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(n_bytes, dtype=torch.uint8, device=dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def reps_of(launch):
        launch()
        torch.cuda.synchronize()
        got = []
        for _ in range(reps):
            a.record()
            launch()
            b.record()
            torch.cuda.synchronize()
            got.append(n_bytes / (a.elapsed_time(b) * 1e-3) / 1e9)
        return {"best": round(max(got), 3), "min": round(min(got), 3),
                "reps": [round(g, 3) for g in got]}

    out = {"hipMemcpyAsync_h2d": reps_of(lambda: dst.copy_(src, non_blocking=True))}
    pair = torch.tensor([0, 0], dtype=torch.int32, device=dev)
    one = torch.tensor([1], dtype=torch.int32, device=dev)
    big = [ctypes.c_void_p(dst.data_ptr()), ctypes.c_void_p(device_address(src)),
           ctypes.c_long(n_bytes)] * 6
    for g in grids:
        def launch(g=g):
            if lib.expert_cache_gather(*big, ctypes.c_void_p(pair.data_ptr()),
                                       ctypes.c_void_p(one.data_ptr()), g, 1, s_ptr):
                raise RuntimeError("gather launch failed")
        out[f"gather_kernel_{g}x1"] = reps_of(launch)
    del src, dst
    peak = max(v["best"] for v in out.values())
    spread = max(v["best"] for v in out.values()) - min(v["min"] for v in out.values())
    log("link peak: " + ", ".join(f"{k} best {v['best']:.2f} (min {v['min']:.2f})"
                                  for k, v in out.items()) + f" GB/s -> {peak:.2f}")
    return peak, {"methods": out, "bytes_per_rep": n_bytes, "spread_GBps": round(spread, 3)}


def _spread(lo, hi, n, length):
    """n segment starts of `length` steps spread evenly over [lo, hi)."""
    n = max(1, n)
    if n == 1 or hi - lo <= length:
        return [lo]
    return sorted({lo + (k * (hi - lo - length)) // (n - 1) for k in range(n)})


def oracle_check(np, ids_np, L, E, S, policy, decay, TP, gpu_nm, gpu_miss, gpu_final):
    """The check of the GPU's trace pass against the oracle, and the oracle's policy timing.

    Timed: the oracle's C policy (oracle/policy.c, one core) over the trace pass from a
    cold start, every layer; the same over up to 16 host threads.

    Checked: the oracle's per-step n_miss and miss lists over the trace pass, and its final
    state, against what the GPU's graph produced (gpu_nm [TP, L], gpu_miss [TP, L, 2S],
    gpu_final the GPU state after step TP)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    rows = [np.ascontiguousarray(ids_np[:TP, l]) for l in range(L)]
    t0 = oracle.now()
    runs = [oracle.run_trace(rows[l], E, S, policy, decay) for l in range(L)]
    policy_us = (oracle.now() - t0) / (TP * L) * 1e6
    # the same policy work spread over host threads, one layer at a time per thread (the C
    # call releases the interpreter lock); layers are independent
    from concurrent.futures import ThreadPoolExecutor
    threads = max(1, min(16, os.cpu_count() or 1, L))
    t0 = oracle.now()
    with ThreadPoolExecutor(threads) as ex:
        par = list(ex.map(lambda l: oracle.run_trace(rows[l], E, S, policy, decay,
                                                     record_miss=True), range(L)))
    policy_par_us = (oracle.now() - t0) / (TP * L) * 1e6

    # the check: per-step n_miss and miss lists, then every final state field
    nm_ok = all(np.array_equal(par[l]["n_miss"], gpu_nm[:, l]) for l in range(L))
    miss_ok = all(np.array_equal(par[l]["miss"], gpu_miss[:, l]) for l in range(L))
    fields = ("table", "map_cold", "slot_expert", "slot_stamp", "step")
    got = {f: gpu_final[f].cpu().numpy() for f in fields}
    state_ok = all(np.array_equal(getattr(runs[l]["final"], f).ravel(), got[f][l].ravel())
                   and np.array_equal(getattr(par[l]["final"], f).ravel(), got[f][l].ravel())
                   for l in range(L) for f in fields)
    log(f"verify: oracle over {TP} steps x {L} layers: per-step n_miss "
        f"{'equal' if nm_ok else 'MISMATCH'}, miss lists {'equal' if miss_ok else 'MISMATCH'}, "
        f"final state {'equal' if state_ok else 'MISMATCH'}")
    check = {"state": state_ok, "n_miss_per_step": nm_ok, "miss_lists_per_step": miss_ok}
    timing = {"policy_us_per_layer_step": round(policy_us, 4),
              "policy_sample": f"trace steps 0..{TP} x {L} layers from a cold start",
              "policy_us_per_layer_step_threads": round(policy_par_us, 4),
              "policy_threads": threads}
    log(f"oracle policy: {policy_us:.3f} us/layer-step (one core), {policy_par_us:.3f} "
        f"us/layer-step over {threads} threads")
    return check, timing


def cpu_baseline(args, torch, np, ids_np, host, slots, bufs, snap, L, E, S, mk, policy, decay,
                 W, policy_timing):
    """The CPU path on this host: the CPU-driven cache over a bounded sample (the first
    cpu_steps timed steps from the timed window's start state): the oracle's C policy
    (oracle/policy.c, one core) decides each layer's misses and each (miss, buffer) is one
    hipMemcpyAsync from pinned host memory into the slot. policy_timing is the oracle's
    policy timing from oracle_check."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    states = []
    for l in range(L):
        s = oracle.State(E, S)
        s.table[:] = snap["table"][l].cpu().numpy()
        s.map_cold[:] = snap["map_cold"][l].cpu().numpy()
        s.slot_expert[:] = snap["slot_expert"][l].cpu().numpy()
        s.slot_stamp[:] = snap["slot_stamp"][l].cpu().numpy()
        s.step[:] = snap["step"][l].cpu().numpy()
        states.append(s)
    B_exp = sum(bufs)
    n = min(args.cpu_steps, ids_np.shape[0] - W)
    torch.cuda.synchronize()
    moved = 0
    t0 = time.perf_counter()
    for t in range(W, W + n):
        for l in range(L):
            s = states[l]
            s.manage(ids_np[t, l], min(E, mk), S, policy, decay)
            for j in range(int(s.n_miss[0])):
                e, sl = int(s.miss[2 * j]), int(s.miss[2 * j + 1])
                for i, b in enumerate(bufs):
                    slots[l][i][sl * b:(sl + 1) * b].copy_(host[l][i][e * b:(e + 1) * b],
                                                           non_blocking=True)
                moved += B_exp
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    hbuf = torch.empty(256 << 20, dtype=torch.uint8, pin_memory=True)
    hsrc = torch.empty(256 << 20, dtype=torch.uint8, pin_memory=True)
    hbuf.copy_(hsrc)
    t1 = time.perf_counter()
    for _ in range(4):
        hbuf.copy_(hsrc)
    host_memcpy = 4 * (256 << 20) / (time.perf_counter() - t1) / 1e9
    log(f"cpu baseline: {n} steps x {L} layers, {moved / 1e9:.2f} GB in {wall:.2f}s -> "
        f"{moved / wall / 1e9:.2f} GB/s; host memcpy {host_memcpy:.1f} GB/s")
    return {"value": round(moved / wall / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"trace steps {W}..{W + n} x {L} layers from the timed steps' start "
                      f"state: C policy (oracle/policy.c) per layer-step, then one "
                      f"hipMemcpyAsync H2D per (miss, buffer)",
            **policy_timing,
            "host_memcpy_GBps": round(host_memcpy, 2),
            "fused_us_per_layer_step": None if args.no_fused else _cpu_fused(np, oracle),
            "pcie_round_trip_us_per_layer_step": _pcie_round_trip(torch),
            "cpu": _cpu_model(), "nproc": os.cpu_count()}


def _pcie_round_trip(torch, n=2000):
    """What a CPU policy path adds per layer-step on top of its own compute: the step's
    routing ids (128 int32) copied to the host and synchronized on, and its outputs (the
    slot ids plus a small miss list, 1 KB) copied back."""
    dev = torch.device("cuda:0")
    ids_d = torch.zeros(128, dtype=torch.int32, device=dev)
    ids_h = torch.empty(128, dtype=torch.int32, pin_memory=True)
    out_h = torch.zeros(256, dtype=torch.int32, pin_memory=True)
    out_d = torch.empty(256, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n):
        ids_h.copy_(ids_d, non_blocking=True)
        torch.cuda.current_stream().synchronize()
        out_d.copy_(out_h, non_blocking=True)
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) / n * 1e6
    log(f"cpu baseline: PCIe round trip of one layer-step's ids and outputs {us:.2f} us")
    return round(us, 3)


def _align_lengths(mk, E, bs):
    """vLLM's moe_align_block_size buffer lengths (kernels/expert_cache.hip:606-609)."""
    L = min(mk * bs, mk + E * (bs - 1)) if mk < E else mk + E * (bs - 1)
    return L, -(-L // bs)


def _fused_routing(np, name):
    from vllm_expert_cache import traces
    w = traces.WORKLOADS[name]
    return w, np.stack([traces.routing(w, l, FUSED_STEPS) for l in range(FUSED_LAYERS)],
                       axis=1)  # [T, layers, mk]


def _cpu_fused(np, oracle):
    """The oracle's fused step (one core) over the fused leg's steps, us per layer-step."""
    out = {}
    for name, S in FUSED_CASES:
        w, ids = _fused_routing(np, name)
        E, mk = w.experts, w.mk
        L, NB = _align_lengths(mk, E, FUSED_BS)
        states = [oracle.State(E, S) for _ in range(FUSED_LAYERS)]
        rows = [np.ascontiguousarray(ids[:, l]) for l in range(FUSED_LAYERS)]
        t0 = oracle.now()
        for l in range(FUSED_LAYERS):
            assert states[l].fused_trace(rows[l], FUSED_BS, L, NB) == 0
        out[name] = round((oracle.now() - t0) / (FUSED_STEPS * FUSED_LAYERS) * 1e6, 3)
    log(f"cpu baseline, fused: {out} us/layer-step (one core)")
    return out


def fused_leg(torch, np, lib, dev, hold):
    """expert_cache_fused per layer-step: FUSED_LAYERS launches captured in one graph,
    replayed for FUSED_STEPS steps of each FUSED_CASES workload from a cold start, the
    step's ids copied into the graph's input first. The kernel is latency-bound; its
    algorithmic bytes per call are the policy step's (ids, state read and written, the
    miss list) plus both align outputs written."""
    keys = ("sorted_hot", "eids_hot", "npad_hot", "sorted_cold", "eids_cold", "npad_cold")
    runs = []
    for name, S in FUSED_CASES:
        w, ids_np = _fused_routing(np, name)
        E, mk, Ly = w.experts, w.mk, FUSED_LAYERS
        L, NB = _align_lengths(mk, E, FUSED_BS)
        sizes = dict(sorted_hot=L, eids_hot=NB, npad_hot=1, sorted_cold=L, eids_cold=NB,
                     npad_cold=1)
        ids_dev = torch.as_tensor(ids_np, device=dev)
        st = Layers(torch, Ly, E, S, dev)
        ids_static = torch.zeros((Ly, mk), dtype=torch.int32, device=dev)
        nm = torch.zeros((Ly,), dtype=torch.int32, device=dev)
        nm_hist = torch.zeros((FUSED_STEPS, Ly), dtype=torch.int32, device=dev)
        outs = {k: torch.zeros((Ly, n), dtype=torch.int32, device=dev) for k, n in sizes.items()}
        args = [(_row(ids_static, l), mk, E, S, min(E, mk), S, st.row("table", l),
                 st.row("map_cold", l), st.row("slot_expert", l), st.row("slot_stamp", l),
                 st.row("routed", l), st.row("step", l), st.row("miss", l),
                 _row(nm, l), FUSED_BS, L, NB, *[_row(outs[k], l) for k in keys])
                for l in range(Ly)]

        def launch(stream):
            c = ctypes.c_void_p(stream.cuda_stream)
            for a in args:
                if lib.expert_cache_fused(*a, c):
                    raise RuntimeError("expert_cache_fused launch failed")

        snap = st.snapshot()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            launch(side)  # warm-up outside capture
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        st.restore(snap)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            launch(torch.cuda.current_stream())
        torch.cuda.synchronize()
        for t in range(FUSED_STEPS):  # inserts per step, untimed
            ids_static.copy_(ids_dev[t], non_blocking=True)
            g.replay()
            nm_hist[t].copy_(nm, non_blocking=True)
        st.restore(snap)
        # steps queued behind stream holds: a step is a few tens of us of GPU work, less
        # than the host takes to queue it, so without the holds the figure would be the
        # host's launch rate

        def enqueue(t):
            ids_static.copy_(ids_dev[t], non_blocking=True)
            g.replay()

        sec = sum(x[2] for x in hold.time(0, FUSED_STEPS, enqueue))
        del g
        us = sec * 1e6 / (FUSED_STEPS * Ly)
        inserts = float(nm_hist.float().mean())
        policy_bytes = 4 * mk + 2 * (8 * E + 12 * S + 8) + 8 * inserts + 4
        out_bytes = 2 * (4 * L + 4 * NB + 4)
        runs.append({"workload": name, "experts": E, "slots": S, "ids_per_step": mk,
                     "block_size": FUSED_BS, "graph_us_per_layer_step": round(us, 3),
                     "algorithmic_bytes_per_call": int(policy_bytes + out_bytes),
                     "achieved_GBps": round((policy_bytes + out_bytes) / (us * 1e3), 3),
                     "inserts_per_layer_step": round(inserts, 4)})
        log(f"fused {name}: E={E} S={S} mk={mk} bs={FUSED_BS}, {us:.2f} us/layer-step in "
            f"graph replay, {int(policy_bytes + out_bytes)} algorithmic bytes per call")
    return {"bound": "latency (one wave, dependent LDS phases)", "layers": FUSED_LAYERS,
            "steps": FUSED_STEPS, "def": "graph replay of one launch per layer, including "
            "the per-step id copy, steps queued in chunks behind stream holds so the host's "
            "launch rate is out of the figure; LRU, cold start. cpu_baseline.fused_us_per_layer_step is "
            "the oracle's fused step in C on one core with the state in host memory: it "
            "leaves out moving each step's ids to the host and the outputs back, which a "
            "CPU path would pay every layer-step", "runs": runs}


def _distinct(np, ids):
    """Distinct expert ids per [..., mk] row, -1 padding not counted."""
    srt = np.sort(ids, axis=-1)
    new = np.ones(srt.shape, bool)
    new[..., 1:] = srt[..., 1:] != srt[..., :-1]
    return (new & (srt >= 0)).sum(-1)


def _row(t, l):
    return ctypes.c_void_p(t.data_ptr() + l * t.stride(0) * t.element_size())


def _row_off(t, l, i):
    return ctypes.c_void_p(t.data_ptr() + (l * t.stride(0) + i) * t.element_size())


def _oracle_prefetch_sequence(np, snap_np, ids, pred, L, E, S, mk, policy, decay, budget):
    """Per layer, from the snapshot's state: for each step t, the oracle's prefetch step of
    pred[t, l] (when pred is given) and then its policy step of ids[t, l], as the prefetch
    leg's graph orders them for that layer. Returns per-layer n_miss [K], miss pairs, the
    prefetch step's n_miss and pairs, and the final state."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    from concurrent.futures import ThreadPoolExecutor

    K = ids.shape[0]

    def layer(l):
        s = oracle.State(E, S)
        for f in ("table", "map_cold", "slot_expert", "slot_stamp", "step", "miss"):
            getattr(s, f)[:] = snap_np[f][l].ravel()
        nm = np.zeros(K, np.int32)
        pn = np.zeros(K, np.int32)
        pairs, pf_pairs = [], []
        for t in range(K):
            if pred is not None:
                assert s.prefetch(pred[t, l], budget) == 0
                pn[t] = s.n_miss[0]
                pf_pairs.append(s.miss[:2 * pn[t]].copy())
            assert s.manage(ids[t, l], min(E, mk), S, policy, decay) == 0
            nm[t] = s.n_miss[0]
            pairs.append(s.miss[:2 * nm[t]].copy())
        return {"n_miss": nm, "pairs": pairs, "pf_n_miss": pn, "pf_pairs": pf_pairs,
                "final": {f: getattr(s, f).copy() for f in
                          ("table", "map_cold", "slot_expert", "slot_stamp", "step")}}

    with ThreadPoolExecutor(max(1, min(16, os.cpu_count() or 1))) as ex:
        return list(ex.map(layer, range(L)))


def _prefetch_matches(np, want, nm, miss, pn, pf_miss, final):
    """The prefetch leg's GPU record (nm [K, L], miss [K, L, 2S], pn / pf_miss likewise or
    None, final state fields [L, ...]) against _oracle_prefetch_sequence."""
    for l, w in enumerate(want):
        if not np.array_equal(w["n_miss"], nm[:, l]):
            return False
        if any(not np.array_equal(p, miss[t, l, :len(p)]) for t, p in enumerate(w["pairs"])):
            return False
        if pn is not None:
            if not np.array_equal(w["pf_n_miss"], pn[:, l]):
                return False
            if any(not np.array_equal(p, pf_miss[t, l, :len(p)])
                   for t, p in enumerate(w["pf_pairs"])):
                return False
        if any(not np.array_equal(w["final"][f].ravel(), final[f][l].ravel()) for f in final):
            return False
    return True


PREFETCH_RUNS = (
    {},                                                     # no prefetch
    {"accuracy": 1.0, "lookahead": 1, "one_launch": False},
    {"accuracy": 1.0, "lookahead": 1},
    {"accuracy": 1.0, "lookahead": 1, "late_fork": True},
    {"accuracy": 1.0, "lookahead": 2},
    {"accuracy": 1.0, "lookahead": 3},
    {"accuracy": 1.0, "lookahead": 4},
    {"accuracy": 1.0, "lookahead": 3, "pair": True},
    {"accuracy": 1.0, "lookahead": 4, "pair": True},
    {"accuracy": 0.8, "lookahead": 1},
    {"accuracy": 0.8, "lookahead": 1, "late_fork": True},
    {"accuracy": 0.8, "lookahead": 2},
    {"accuracy": 0.8, "lookahead": 3},
    {"accuracy": 0.8, "lookahead": 1, "budget": 1},
    {"accuracy": 0.8, "lookahead": 1, "errors": "routed"},
    {"accuracy": 0.8, "lookahead": 1, "errors": "routed", "late_fork": True},
    {"accuracy": 0.8, "lookahead": 2, "errors": "routed"},
    {"accuracy": 0.8, "lookahead": 3, "errors": "routed"},
)


def _predictions(np, ids_np, W, K, E, q, errors):
    """The true routing of steps W..W+K with each id replaced, with probability 1 - q, by a
    wrong guess: a uniformly random expert ("uniform"), or an expert the same layer routes
    at a random step of the trace ("routed": a plausible alternative, drawn as often as the
    layer routes it)."""
    rng = np.random.default_rng(int(q * 1000) + (1 if errors == "routed" else 0))
    pred = ids_np[W:W + K].copy()
    wrong = (rng.random(pred.shape) >= q) & (pred >= 0)
    n = int(wrong.sum())
    if errors == "uniform":
        pred[wrong] = rng.integers(0, E, n)
    else:
        layer = np.nonzero(wrong)[1]
        pred[wrong] = ids_np[rng.integers(0, ids_np.shape[0], n), layer,
                             rng.integers(0, ids_np.shape[2], n)]
    return pred


def prefetch_leg(torch, np, lib, ids_np, ids_dev, g_args, snap, L, E, S, mk, policy, decay,
                 W, T, B_exp, chunks, lanes, dev, peak, slots, content, bufs, window=1024,
                 compute=(0, 50), runs=PREFETCH_RUNS, pf_chunks=None):
    """Prefetch over trace steps W..T, every run from the same start state (the snapshot
    `snap` taken at step W of the trace pass), as one captured graph per decode step.

    With a lookahead of d layers:
      d = 0 (no prefetch): per layer l, manage+remap(l), gather(l), compute(l);
      d >= 1: layers 0..d-1 prefetched first, then per layer l the prefetch step of layer
              l+d and manage+remap(l) -- two launches (expert_cache_prefetch, then
              expert_cache_manage_remap) or one (expert_cache_manage_remap_prefetch) --,
              a wait for layer l's prefetch copy, gather(l) of what is still missing,
              compute(l). The copy of layer l+d's prefetched experts
              (expert_cache_gather_live, on a side stream) forks right after the policy
              launch (the default, as ExpertSlotCache does) or, with "late_fork", after
              gather(l), so that it does not share the host link with gather(l); with
              "pair", after every second policy launch, carrying the copies of the two
              layers prefetched since (half the cross-stream edges; half the copies start
              a layer later).
    The real step of a layer settles its pending prefetch installs: routed ones stay, the
    others are dropped, and their live copy stops.

    compute(l) stands in for the layer's attention and expert GEMMs: a spin of C us on one
    CU (C = 0: no compute, so prefetch has nothing to hide behind). Predictions come from
    _predictions; accuracy 1.0 is an upper bound no real predictor reaches. Each run is a
    dict of accuracy (absent: no prefetch), lookahead, one_launch (default True), late_fork
    (default False), pair (default False), budget (inserts per prefetch step, default S) and
    errors ("uniform", the default, or "routed").

    Checked: every run's per-step n_miss and miss list of each layer's real step and of its
    prefetch step, and the final state, against the oracle's prefetch and policy steps
    (oracle/policy.c) called in the order the graph makes them per layer; and, in the first
    run of each predictor accuracy, every resident slot's bytes at the end, the slots having
    been re-gathered from the snapshot's residents before the run."""
    K = min(window, T - W)
    i32 = torch.int32
    tt, ll = np.meshgrid(np.arange(K), np.arange(L), indexing="ij")
    routed = np.zeros((K, L, E), bool)
    for i in range(mk):
        v = ids_np[W:W + K, :, i]
        m = v >= 0  # -1 pads a recorded trace
        routed[tt[m], ll[m], v[m]] = True
    distinct = int(routed.sum())

    # spin cycles per microsecond, measured
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    torch.cuda._sleep(int(2e6))
    b.record()
    torch.cuda.synchronize()
    cyc_per_us = 2e6 / (a.elapsed_time(b) * 1e3)

    st = Layers(torch, L, E, S, dev)
    pf_miss = torch.zeros((L, 2 * S), dtype=i32, device=dev)
    pf_nm = torch.zeros((L,), dtype=i32, device=dev)
    ids_static = torch.zeros((L, mk), dtype=i32, device=dev)
    pred_static = torch.zeros((L, mk), dtype=i32, device=dev)
    out_static = torch.zeros((L, mk), dtype=i32, device=dev)
    nm_static = st.n_miss
    nm_hist = torch.zeros((K, L), dtype=i32, device=dev)
    pf_hist = torch.zeros((K, L), dtype=i32, device=dev)
    pf_miss_hist = torch.zeros((K, L, 2 * S), dtype=i32, device=dev)
    miss_hist = torch.zeros((K, L, 2 * S), dtype=i32, device=dev)
    snap_np = {f: snap[f].cpu().numpy() for f in ("table", "map_cold", "slot_expert",
                                                  "slot_stamp", "step", "miss")}
    expected = {}  # oracle sequences by (predictor, errors, budget)
    checks = []
    slot_checked = set()

    def regather():
        """Slot bytes consistent with the snapshot: every resident (expert, slot) copied."""
        rec = torch.zeros((L, 1 + 2 * S), dtype=i32)
        for l in range(L):
            se = snap_np["slot_expert"][l]
            res = np.nonzero(se >= 0)[0]
            rec[l, 0] = len(res)
            rec[l, 1:1 + 2 * len(res):2] = torch.as_tensor(se[res])
            rec[l, 2:2 + 2 * len(res):2] = torch.as_tensor(res.astype(np.int32))
        rec = rec.to(dev)
        s0 = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for l in range(L):
            if lib.expert_cache_gather(*g_args[l][:18], _row_off(rec, l, 1), _row(rec, l),
                                       chunks, lanes, s0):
                raise RuntimeError("re-gather launch failed")
        torch.cuda.synchronize()
    side = torch.cuda.Stream(dev)
    done = [torch.cuda.Event() for _ in range(L)]
    m_args = [(_row(ids_static, l), 4, mk, E, S, min(E, mk), S, st.row("table", l),
               st.row("map_cold", l), st.row("slot_expert", l), st.row("slot_stamp", l),
               st.row("routed", l), st.row("step", l), st.row("miss", l),
               _row(nm_static, l), policy, decay, _row(out_static, l)) for l in range(L)]
    p_args = [(_row(pred_static, l), mk, E, S, S, st.row("table", l), st.row("map_cold", l),
               st.row("slot_expert", l), st.row("slot_stamp", l), st.row("routed", l),
               _row(pf_miss, l), _row(pf_nm, l)) for l in range(L)]
    gp_args = [tuple(g_args[l][:18]) + (_row(pf_miss, l), _row(pf_nm, l),
                                        st.row("slot_expert", l), pf_chunks or chunks, 1)
               for l in range(L)]
    gr_args = [tuple(g_args[l][:18]) + (st.row("miss", l), _row(nm_static, l), chunks, lanes)
               for l in range(L)]

    def launch(cur, la, one, late, budget, spin, pair=False):
        c = ctypes.c_void_p(cur.cuda_stream)
        sd = ctypes.c_void_p(side.cuda_stream)
        pa = [a[:4] + (budget,) + a[5:] for a in p_args]
        held = []  # with pair: prefetched layers whose copy waits for the next fork

        def copy(l):
            if pair and l >= la:
                held.append(l)
                if len(held) < 2 and l < L - 1:
                    return 0
            side.wait_stream(cur)
            rc = 0
            for m in (held if pair and l >= la else [l]):
                rc |= lib.expert_cache_gather_live(*gp_args[m], sd)
                done[m].record(side)
            held.clear()
            return rc

        rc = 0
        for j in range(min(la, L)):
            rc |= lib.expert_cache_prefetch(*pa[j], c) | copy(j)
        for l in range(L):
            n = l + la
            fork = None
            if la and n < L and one:
                rc |= lib.expert_cache_manage_remap_prefetch(*m_args[l], _row(pred_static, n),
                                                             mk, budget, *pa[n][5:], c)
                fork = n
            elif la and n < L:
                rc |= lib.expert_cache_prefetch(*pa[n], c)
                fork = n
                if not late:
                    rc |= copy(n)
                    fork = None
                rc |= lib.expert_cache_manage_remap(*m_args[l], c)
            else:
                rc |= lib.expert_cache_manage_remap(*m_args[l], c)
            if fork is not None and not late:
                rc |= copy(fork)
                fork = None
            if la:
                cur.wait_event(done[l])
            rc |= lib.expert_cache_gather(*gr_args[l], c)
            if fork is not None:
                rc |= copy(fork)
            if spin:
                torch.cuda._sleep(spin)
        if rc:
            raise RuntimeError(f"decode step launch failed rc={rc}")

    out = []
    base_ms = {}
    for C in compute:
        for run in runs:
            q = run.get("accuracy")
            la = run.get("lookahead", 0) if q is not None else 0
            one, late = run.get("one_launch", True), run.get("late_fork", False)
            pair = run.get("pair", False)
            budget = run.get("budget") or S
            errors = run.get("errors", "uniform")
            pred = None if q is None else (ids_np[W:W + K].copy() if q >= 1.0 else
                                           _predictions(np, ids_np, W, K, E, q, errors))
            if pred is not None:
                pred_dev = torch.as_tensor(np.ascontiguousarray(pred), device=dev)
            key = (q, errors if q is not None and q < 1.0 else None,
                   budget if q is not None else None)
            check_slots = key[:2] not in slot_checked
            slot_checked.add(key[:2])
            st.restore(snap)
            if check_slots:
                regather()
            pf_nm.zero_()
            pf_hist.zero_()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                launch(torch.cuda.current_stream(), la, one, late, budget, int(C * cyc_per_us),
                       pair)
            torch.cuda.synchronize()
            wall0 = time.perf_counter()
            a.record()
            for t in range(K):
                ids_static.copy_(ids_dev[W + t], non_blocking=True)
                if pred is not None:
                    pred_static.copy_(pred_dev[t], non_blocking=True)
                g.replay()
                nm_hist[t].copy_(nm_static, non_blocking=True)
                miss_hist[t].copy_(st.miss, non_blocking=True)
                if pred is not None:
                    pf_hist[t].copy_(pf_nm, non_blocking=True)
                    pf_miss_hist[t].copy_(pf_miss, non_blocking=True)
            b.record()
            torch.cuda.synchronize()
            elapsed = max(time.perf_counter() - wall0, a.elapsed_time(b) * 1e-3)
            del g
            nm, pn = nm_hist.cpu().numpy(), pf_hist.cpu().numpy()
            if key not in expected:
                expected[key] = _oracle_prefetch_sequence(
                    np, snap_np, ids_np[W:W + K], pred, L, E, S, mk, policy, decay, budget)
            ok = _prefetch_matches(np, expected[key], nm, miss_hist.cpu().numpy(),
                                   pn if pred is not None else None,
                                   pf_miss_hist.cpu().numpy() if pred is not None else None,
                                   {f: getattr(st, f).cpu().numpy() for f in
                                    ("table", "map_cold", "slot_expert", "slot_stamp", "step")})
            slots_ok = None
            if check_slots:
                from vllm_expert_cache import traces
                slots_ok = all(traces.slots_match(slots[l][b], st.slot_expert[l], content[l],
                                                  b, nb)[0]
                               for l in range(L) for b, nb in enumerate(bufs))
            checks.append({"oracle": ok, "slot_bytes": slots_ok})
            used = 0
            if pred is not None:
                fetched = pf_miss_hist.cpu().numpy()[..., 0::2]
                valid = np.arange(S)[None, None, :] < pn[..., None]
                used = int((routed[tt[..., None], ll[..., None], np.where(valid, fetched, 0)]
                            & valid).sum())
            ms = 1e3 * elapsed / K
            if q is None:
                base_ms[C] = ms
            useful = (int(nm.sum()) + used) * B_exp / elapsed / 1e9
            out.append({"compute_us_per_layer": C, "predictor_accuracy": q,
                        "prediction_errors": errors if q is not None and q < 1.0 else None,
                        "lookahead_layers": la, "one_launch": one if la else None,
                        "copy_fork": (None if not la else
                                      "after the layer's gather" if late else
                                      "after every second policy launch, two layers' "
                                      "copies" if pair else "after the policy launch"),
                        "insert_budget": budget if q is not None else None,
                        "ms_per_step": round(ms, 4),
                        "speedup_vs_no_prefetch": round(base_ms[C] / ms, 4),
                        "useful_GBps": round(useful, 3),
                        "prefetch_inserts": int(pn.sum()), "prefetch_used": used,
                        "prefetch_dropped": int(pn.sum()) - used,
                        "critical_path_inserts": int(nm.sum()),
                        "real_step_hit_rate": round(1.0 - float(nm.sum()) / distinct, 5)})
            desc = "none" if q is None else (
                f"{q} ({errors} errors), lookahead {la}"
                f"{', one launch' if one else ', two launches'}"
                f"{', copy forked after the gather' if late else ''}"
                f"{', copies forked two layers at a time' if pair else ''}"
                f"{f', budget {budget}' if budget < S else ''}")
            log(f"prefetch leg, compute {C} us/layer, predictor {desc}: {ms:.3f} ms/step "
                f"({base_ms[C] / ms:.3f}x), {int(pn.sum())} prefetched ({used} used), "
                f"{int(nm.sum())} on the critical path; oracle {'equal' if ok else 'MISMATCH'}"
                f"{'' if slots_ok is None else ', slot bytes ' + ('equal' if slots_ok else 'MISMATCH')}")
    return {"window_steps": K, "trace_steps": [W, W + K],
            "spin_cycles_per_us": round(cyc_per_us, 1),
            "copy_grid": [pf_chunks or chunks, 1],
            "def": "useful_GBps counts the experts a step needed (critical-path inserts plus "
                   "prefetched experts that were routed), not the partial copies of dropped "
                   "predictions", "runs": out,
            "verified": {"oracle_runs": sum(c["oracle"] for c in checks),
                         "runs": len(checks),
                         "slot_byte_runs": sum(c["slot_bytes"] is True for c in checks),
                         "slot_byte_checks": sum(c["slot_bytes"] is not None for c in checks),
                         "all": all(c["oracle"] and c["slot_bytes"] is not False
                                    for c in checks),
                         "def": "per run: each layer's per-step n_miss and miss list (real "
                                "and prefetch steps) and final state against the oracle's "
                                "prefetch and policy steps in the graph's per-layer order; "
                                "in the first run of each predictor, every resident slot's "
                                "bytes after the run (slots re-gathered from the start "
                                "state's residents first)"}}


SWEEP_CHUNK = 16  # decode steps per captured graph in the hit-rate sweep


def hit_rate_sweep(torch, np, lib, w, ids_np, ids_dev, L, E, mk, decay, dev, hold):
    """Hit rate per slot budget and policy over the whole trace from a cold start, on the
    GPU policy kernel (no gather: hit rate and gather volume depend only on the policy).

    SWEEP_CHUNK decode steps are captured in one graph of SWEEP_CHUNK x L policy+remap
    launches, each reading its step's ids from a window buffer and writing its n_miss into a
    window of the history; per chunk the host copies the window's ids in, replays, and
    copies the n_miss window out. Chunks are queued behind stream holds, so the graph's time
    per layer is the policy launches back to back (kernel plus graph node gap), with two
    small copies per SWEEP_CHUNK steps, not the host's queueing rate."""
    T = ids_np.shape[0]
    C = SWEEP_CHUNK
    distinct = _distinct(np, ids_np)  # [T, L]
    Tp = -(-T // C) * C  # padded to whole chunks with empty steps (-1 ids: nothing routed)
    ids_pad = torch.full((Tp, L, mk), -1, dtype=torch.int32, device=dev)
    ids_pad[:T].copy_(ids_dev)
    out = []
    for S in w.slots:
        if mk > S:
            out.append({"slots": S, "served_steps": 0,
                        "note": "tokens x top_k > slots: every step reads through"})
            continue
        for pol_name in w.policies:
            pol = 1 if pol_name == "lfu" else 0
            st = Layers(torch, L, E, S, dev)
            ids_win = torch.zeros((C, L, mk), dtype=torch.int32, device=dev)
            out_static = torch.zeros((L, mk), dtype=torch.int32, device=dev)
            nm_win = torch.zeros((C, L), dtype=torch.int32, device=dev)
            nm_hist = torch.zeros((Tp, L), dtype=torch.int32, device=dev)
            args_l = [[(_row(ids_win[i], l), 4, mk, E, S, min(E, mk), S, st.row("table", l),
                        st.row("map_cold", l), st.row("slot_expert", l),
                        st.row("slot_stamp", l), st.row("routed", l), st.row("step", l),
                        st.row("miss", l), _row(nm_win[i], l), pol, decay,
                        _row(out_static, l)) for l in range(L)] for i in range(C)]

            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                for i in range(C):
                    for l in range(L):
                        if lib.expert_cache_manage_remap(*args_l[i][l], sp):
                            raise RuntimeError("manage launch failed")
            torch.cuda.synchronize()

            def enqueue(k):
                ids_win.copy_(ids_pad[k * C:(k + 1) * C], non_blocking=True)
                g.replay()
                nm_hist[k * C:(k + 1) * C].copy_(nm_win, non_blocking=True)

            sec = sum(x[2] for x in hold.time(0, Tp // C, enqueue, chunk=4))
            nm = nm_hist[:T].cpu().numpy()
            # a padded step routes nothing, so it inserts nothing; its launches are timed
            # with the rest (at most C - 1 steps of T)
            per_layer = 1.0 - nm.sum(0) / distinct.sum(0)
            out.append({"slots": S, "policy": pol_name, "steps": T,
                        "hit_rate": round(float(1.0 - nm.sum() / distinct.sum()), 5),
                        "per_layer_hit_rate_min": round(float(per_layer.min()), 5),
                        "per_layer_hit_rate_max": round(float(per_layer.max()), 5),
                        "inserts": int(nm.sum()),
                        "gather_volume_GB": round(float(nm.sum()) * w.bytes_per_expert / 1e9, 2),
                        "graph_us_per_layer": round(sec * 1e6 / (Tp * L), 3)})
            log(f"hit-rate sweep: S={S} {pol_name}: {out[-1]['hit_rate']} "
                f"(layers {out[-1]['per_layer_hit_rate_min']}..{out[-1]['per_layer_hit_rate_max']}), "
                f"{out[-1]['gather_volume_GB']} GB, {out[-1]['graph_us_per_layer']} us/layer")
            del g
    return out


def _traffic():
    """Measured bytes per one-miss gather launch (rocprofv3 FETCH_SIZE / WRITE_SIZE,
    calibrated on a plain copy), from the committed profile summary; None if absent."""
    p = ROOT / "profiles" / "gather_k-traffic-48-layer-e128.json"
    try:
        t = json.loads(p.read_text())
    except (OSError, ValueError):
        return None
    return {"bytes_per_launch": t["fetch_bytes_per_launch"] + t["write_bytes_per_launch"],
            "launch": "one expert (4,732,928 B) per launch",
            "fetch_bytes_per_miss": t["fetch_bytes_per_launch"],
            "write_bytes_per_miss": t["write_bytes_per_launch"],
            "algorithmic_bytes_per_miss": t["algorithmic_bytes_per_launch"],
            "algorithmic_read_plus_write": 2 * t["algorithmic_bytes_per_launch"],
            "fetch_over_algorithmic": t["fetch_over_algorithmic"],
            "source": f"profiles/{p.name}"}


def _manage_counters():
    """Hardware counters per policy+remap call (rocprofv3, calibrated), back to back and in
    the decode loop, from the committed profile summary; None if absent."""
    p = ROOT / "profiles" / "manage_k-counters-48-layer-e128.json"
    try:
        j = json.loads(p.read_text())
        t, c = j["per_call"], j["in_chain"]
    except (OSError, ValueError, KeyError):
        return None
    return {"hbm_bytes_read": c["hbm_fetch_bytes"], "hbm_bytes_written": c["hbm_write_bytes"],
            "hbm_GBps": c["hbm_GBps"], "lds_instructions": c["SQ_INSTS_LDS"],
            "lds_GBps_estimate": c["lds_GBps_estimate"],
            "kernel_us": c["kernel_us_by_clock_stamps"],
            "wave_cycles": c["SQ_WAVE_CYCLES"],
            "back_to_back": {"hbm_bytes_read": t["hbm_fetch_bytes"],
                             "hbm_bytes_written": t["hbm_write_bytes"],
                             "wave_cycles": t["SQ_WAVE_CYCLES"],
                             "profiler_duration_us": t["duration_us"]},
            "profiler_duration_us_in_chain": c["duration_us"],
            "def": "per call in the decode loop (in_chain of the source); GB/s over the "
                   "kernel's own run time in the decode graph (clock stamps)",
            "source": f"profiles/{p.name}"}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


if __name__ == "__main__":
    main()
