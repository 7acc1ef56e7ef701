"""Writes tests/golden/reference_policy_suites.npz: the reference's own kernels
(kernels/expert_cache.hip, compiled unchanged into oracle/_ref by `build()`), run on one
GPU:
  * the policy kernel over the routing of the reference's five policy suites
    (tests/test_policy.py:200-221, generated with this repository's seeds), both policies;
  * the fused kernel (LRU step + both moe_align_block_size outputs) over 64 steps of three
    workloads at block size 16, and 80 steps of a small case at block size 3 with padding
    and out-of-range ids. Outputs are preset to -7 before each step, so a position the
    kernel leaves unwritten would show.

Recorded per suite and policy, after every step: n_miss, the whole miss buffer (the
reference also writes miss[2j] for counted inserts it could not place), and a SHA-256 of
the full state (table | map_cold | slot_expert | slot_stamp | step, int32 words);
the final state in full. Inputs (routing ids, warm-start experts, max_distinct,
max_inserts) are stored beside them, so the fixture stands alone.

Run from the repository root on a GPU, after build():  python tests/golden/make_reference_vectors.py OUT
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT / "tests"), str(ROOT / "oracle"), str(ROOT / "vllm-expert-cache_amd")]

import gpu_util as gu  # noqa: E402
from test_oracle import _suite_traces, align_lengths  # noqa: E402
from vllm_expert_cache import traces  # noqa: E402

FUSED_KEYS = ("sorted_hot", "eids_hot", "npad_hot", "sorted_cold", "eids_cold", "npad_cold")


def fused_cases():
    """name, E, S, bs, ids[T, mk]"""
    out = []
    for name, S in (("48-layer-e128", 64), ("48-layer-e128-batch4", 48),
                    ("8-layer-e256-fp8", 128)):
        w = traces.WORKLOADS[name]
        out.append((f"fused-{name}", w.experts, S, 16, traces.routing(w, 0, 64)))
    rng = np.random.default_rng(5)
    out.append(("fused-small-bs3", 32, 8, 3, rng.integers(-2, 34, size=(80, 6))))
    return out


def fused_run(h, arrays, name, E, S, bs, ids):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, mk = ids.shape
    L, NB = align_lengths(mk, E, bs)
    sizes = dict(sorted_hot=L, eids_hot=NB, npad_hot=1, sorted_cold=L, eids_cold=NB,
                 npad_cold=1)
    st = gu.Layers(1, E, S)
    outs = {k: torch.zeros(n, dtype=torch.int32, device=gu.DEV) for k, n in sizes.items()}
    d_ids = torch.as_tensor(ids, device=gu.DEV)
    nm = np.zeros(T, np.int32)
    digests = []
    for t in range(T):
        for o in outs.values():
            o.fill_(-7)
        assert h.expert_cache_fused(
            gu.ptr(d_ids[t]), mk, E, S, min(E, mk), S, st.row("table", 0),
            st.row("map_cold", 0), st.row("slot_expert", 0), st.row("slot_stamp", 0),
            st.row("routed", 0), st.row("step", 0), st.row("miss", 0), st.row("n_miss", 0),
            bs, L, NB, *[gu.ptr(outs[k]) for k in FUSED_KEYS], gu.stream()) == 0
        torch.cuda.synchronize()
        nm[t] = int(st.n_miss[0, 0])
        blob = np.concatenate([outs[k].cpu().numpy() for k in FUSED_KEYS] +
                              [st.state_words()[0].cpu().numpy()]).astype(np.int32)
        digests.append(hashlib.sha256(blob.tobytes()).digest())
    arrays[f"{name}/ids"] = ids.astype(np.int16)
    arrays[f"{name}/shape"] = np.array([E, S, bs, L, NB], np.int32)
    arrays[f"{name}/n_miss"] = nm
    arrays[f"{name}/digest"] = np.frombuffer(b"".join(digests), np.uint8).reshape(T, 32)
    for k in FUSED_KEYS:
        arrays[f"{name}/last/{k}"] = outs[k].cpu().numpy().astype(np.int32)
    arrays[f"{name}/final"] = st.state_words()[0].cpu().numpy().astype(np.int32)
    print(f"{name}: {T} steps, {int(nm.sum())} inserts", flush=True)

DECAY = 8


def main(out: str) -> None:
    h = gu.ref_lib()
    if h is None:
        raise SystemExit("oracle/_ref/libexpertcache_ref.so is missing: run build() where the "
                         "reference tree is mounted")
    arrays = {}
    names = []
    for name, E, S, ids, md, mi in _suite_traces():
        hot = np.array(sorted(np.random.default_rng(1).choice(E, S, replace=False).tolist()),
                       np.int32)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        arrays[f"{name}/ids"] = ids.astype(np.int16)
        arrays[f"{name}/hot"] = hot
        arrays[f"{name}/shape"] = np.array([E, S, md, mi], np.int32)
        for policy in (0, 1):
            key = f"{name}/p{policy}"
            st = gu.Layers(1, E, S, miss_cap=mi, hot=hot.tolist())
            d_ids = torch.as_tensor(ids, device=gu.DEV)
            T, mk = ids.shape
            nm = np.zeros(T, np.int32)
            miss = np.zeros((T, 2 * mi), np.int16)
            digests = []
            for t in range(T):
                assert gu.manage_call(h, st, 0, gu.ptr(d_ids[t]), mk, md, mi, policy,
                                      DECAY) == 0
                torch.cuda.synchronize()
                nm[t] = int(st.n_miss[0, 0])
                miss[t] = st.miss[0].cpu().numpy().astype(np.int16)
                words = st.state_words()[0].cpu().numpy().astype(np.int32)
                digests.append(hashlib.sha256(words.tobytes()).digest())
            arrays[f"{key}/n_miss"] = nm
            arrays[f"{key}/miss"] = miss
            arrays[f"{key}/digest"] = np.frombuffer(b"".join(digests), np.uint8).reshape(T, 32)
            arrays[f"{key}/final"] = st.state_words()[0].cpu().numpy().astype(np.int32)
            names.append(key)
            print(f"{key}: {T} steps, {int(nm.sum())} inserts", flush=True)
    for name, E, S, bs, ids in fused_cases():
        fused_run(h, arrays, name, E, S, bs, ids)
    arrays["meta/decay"] = np.array([DECAY], np.int32)
    np.savez_compressed(out, **arrays)
    print(f"wrote {out} ({Path(out).stat().st_size} bytes)", flush=True)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else str(ROOT / "tests" / "golden" /
                                                   "reference_policy_suites.npz"))
