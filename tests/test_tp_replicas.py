"""Tensor-parallel replicas keep identical caches with no communication.

Each rank of a TP group runs its own cache on the same routing (vllm_expert_cache/cache.py
:14-15 of the reference). The policy step is deterministic -- misses in id order, victims by
a total order, disjoint installs, no atomics -- so every rank's state must match bit for bit
after any number of steps. Two processes run the trace independently and compare only a
digest of their final state over gloo (CPU tensors), once, at the end.

The CPU variant runs the oracle in each rank; the GPU variant runs the HIP kernels, both
ranks on cuda:0.
"""
from __future__ import annotations

import hashlib
import os
import socket
import sys

import numpy as np
import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _digest(arrays) -> torch.Tensor:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return torch.tensor(list(h.digest()), dtype=torch.uint8)


def _rank_main(rank: int, world: int, port: int, use_gpu: bool, q):
    try:
        for p in ("vllm-expert-cache_amd", "oracle", "tests"):
            sys.path.insert(0, os.path.join(ROOT, p))
        os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
        dist.init_process_group("gloo", rank=rank, world_size=world)
        from vllm_expert_cache import traces

        w = traces.WORKLOADS["48-layer-e128"]
        ids = np.stack([traces.routing(w, l, 512) for l in range(8)], axis=1)
        if use_gpu:
            import gpu_util as gu

            r = gu.run_trace(gu.lib(), ids, w.experts, 32, 1, fused_remap=True,
                             record_state=False)
            st = r["final"]
            arrays = [t.cpu().numpy() for t in (st.table, st.map_cold, st.slot_expert,
                                                  st.slot_stamp, st.step)]
            arrays += [r["n_miss"], r["miss"], r["out"]]
            inserts = int(r["n_miss"][r["n_miss"] > 0].sum())
        else:
            import oracle

            arrays, inserts = [], 0
            for l in range(ids.shape[1]):
                r = oracle.run_trace(np.ascontiguousarray(ids[:, l]), w.experts, 32, 1,
                                     record_miss=True)
                f = r["final"]
                arrays += [f.table, f.map_cold, f.slot_expert, f.slot_stamp, f.step,
                           r["n_miss"], r["miss"]]
                inserts += int(r["n_miss"][r["n_miss"] > 0].sum())
        mine = _digest(arrays)
        got = [torch.zeros_like(mine) for _ in range(world)]
        dist.all_gather(got, mine)
        q.put((rank, all(torch.equal(g, got[0]) for g in got), inserts))
        dist.destroy_process_group()
    except Exception as e:  # report to the parent instead of hanging it
        q.put((rank, repr(e), None))


def _run(use_gpu: bool):
    ctx = mp.get_context("spawn")
    q = ctx.Queue()
    port = _free_port()
    procs = [ctx.Process(target=_rank_main, args=(r, 2, port, use_gpu, q)) for r in range(2)]
    for p in procs:
        p.start()
    results = [q.get(timeout=240) for _ in procs]
    for p in procs:
        p.join(timeout=60)
        assert p.exitcode == 0, p.exitcode
    for rank, same, inserts in results:
        assert same is True, (rank, same)
        assert inserts is not None and inserts > 0


def test_replicas_identical_cpu():
    _run(use_gpu=False)


@pytest.mark.gpu
def test_replicas_identical_gpu():
    _run(use_gpu=True)
