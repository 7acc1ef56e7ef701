"""Policy-step parity on the GPU: the HIP manage kernels against the oracle, bit-exact,
on every field of every step (n_miss, the miss buffer, table, map_cold, slot_expert,
slot_stamp, step) and, for the fused entry point, the remapped slot ids.

Also run: the reference's published insert counts through the GPU kernels, the reference's
five policy suites (warm start, insert cap, read-through gate, padding rows), and the
reference's own kernel (compiled from kernels/expert_cache.hip into oracle/_ref) on the same
traces, which must agree with the oracle too.
"""
from __future__ import annotations

import time

import numpy as np
import pytest
import torch

import gpu_util as gu
import kat_traces
import oracle
from vllm_expert_cache import traces

pytestmark = pytest.mark.gpu

LRU, LFU = 0, 1
POLICY = {"lfu": LFU, "lru": LRU}


def _assert_same(got: dict, want: dict, keys, tag):
    for k in keys:
        a, b = got[k], want[k]
        assert a.shape == b.shape, (tag, k, a.shape, b.shape)
        d = gu.first_diff(a, b)
        assert d is None, f"{tag}: {k} differs first at {d}: {a[d]} != {b[d]}"


def _expected_remap(ids: np.ndarray, state: np.ndarray, E: int) -> np.ndarray:
    """out[t, l, i] = table after step t of layer l, at ids[t, l, i]."""
    table = state[..., :E]
    return np.take_along_axis(table, ids.astype(np.int64), axis=-1).astype(np.int32)


def _workload_cases():
    cases = []
    for name in ("48-layer-e128", "48-layer-e128-batch4", "8-layer-e8-bf16", "8-layer-e256-fp8"):
        w = traces.WORKLOADS[name]
        for s in w.slots:
            for p in w.policies:
                cases.append(pytest.param(name, s, p, id=f"{name}-S{s}-{p}"))
    return cases


@pytest.mark.parametrize("name,slots,policy", _workload_cases())
def test_workload_parity_full_trace(name, slots, policy):
    """The product entry point (manage + fused remap) over every layer and step."""
    w = traces.WORKLOADS[name]
    ids = traces.routing_all_layers(w)
    t0 = time.time()
    got = gu.run_trace(gu.lib(), ids, w.experts, slots, POLICY[policy], fused_remap=True)
    t1 = time.time()
    want = gu.oracle_trace(ids, w.experts, slots, POLICY[policy])
    print(f"{name} S={slots} {policy}: {ids.shape[0]}x{ids.shape[1]} layer-steps, "
          f"gpu {t1 - t0:.1f}s oracle {time.time() - t1:.1f}s, "
          f"inserts {int(want['n_miss'][want['n_miss'] > 0].sum())}", flush=True)
    _assert_same(got, want, ("n_miss", "miss", "state"), name)
    if ids.shape[2] <= slots:
        _assert_same({"out": got["out"]}, {"out": _expected_remap(ids, want["state"],
                                                                   w.experts)}, ("out",), name)
    else:
        assert (got["out"] == -9).all()  # never served: remap never ran


@pytest.mark.parametrize("policy", ["lfu", "lru"])
def test_manage_entry_point_parity(policy):
    """expert_cache_manage (the reference's own entry point) on 48 layers x 1024 steps."""
    w = traces.WORKLOADS["48-layer-e128"]
    ids = traces.routing_all_layers(w, steps=1024)
    got = gu.run_trace(gu.lib(), ids, w.experts, 64, POLICY[policy])
    want = gu.oracle_trace(ids, w.experts, 64, POLICY[policy])
    _assert_same(got, want, ("n_miss", "miss", "state"), "manage")


@pytest.mark.parametrize("rule", ["manage", "manage_remap", "reference"])
@pytest.mark.parametrize("key", sorted(kat_traces.KAT), ids=lambda k: f"{k[0]}-S{k[1]}")
def test_published_insert_counts_on_gpu(key, rule):
    h = gu.ref_lib() if rule == "reference" else gu.lib()
    if h is None:
        pytest.skip("reference library not built")
    workload, slots = key
    ids = kat_traces.trace(workload)[:, None, :]
    for policy, want in zip((LRU, LFU), kat_traces.KAT[key]):
        got = gu.run_trace(h, ids, kat_traces.E, slots, policy,
                           fused_remap=(rule == "manage_remap"), record_state=False)
        assert int(got["n_miss"].sum()) == want, (workload, slots, policy)


def _suites():
    """The reference's policy suites (tests/test_policy.py:202-221) with our seeds:
    name, E, S, ids[T, mk], max_distinct, max_inserts."""
    rng = np.random.default_rng(0)
    zipf = np.arange(1, 513, dtype=float) ** -1.1
    zipf /= zipf.sum()
    padded = rng.choice(64, size=(120, 4, 10))
    padded[:, 2:] = -1
    return [
        ("tiny-churn", 32, 8, rng.choice(32, size=(200, 10)), 8, 8),
        ("skewed-512", 512, 257, np.stack([np.concatenate(
            [rng.choice(512, 10, replace=False, p=zipf) for _ in range(5)])
            for _ in range(300)]), 128, 64),
        ("insert-capped", 128, 32, rng.choice(128, size=(150, 80)), 128, 4),
        ("read-through", 128, 32, rng.choice(128, size=(60, 160)), 8, 16),
        ("padded-rows", 64, 16, padded.reshape(120, 40), 64, 16),
        ("e1024-s1024", 1024, 1024, rng.choice(1024, size=(60, 600)), 1024, 1024),
        ("e5000-s300", 5000, 300, rng.choice(5000, size=(40, 400)), 400, 300),
    ]


def _oracle_steps(ids, E, S, md, mi, policy, decay, hot):
    st = oracle.State(E, S, hot, miss_cap=mi)
    T = ids.shape[0]
    nm = np.zeros((T, 1), np.int32)
    miss = np.zeros((T, 1, 2 * mi), np.int32)
    state = np.zeros((T, 1, oracle.state_words(E, S)), np.int32)
    for t in range(T):
        assert st.manage(ids[t], md, mi, policy, decay) == 0
        nm[t, 0] = st.n_miss[0]
        miss[t, 0] = st.miss
        state[t, 0] = np.concatenate([st.table, st.map_cold, st.slot_expert,
                                      st.slot_stamp.view(np.int32), st.step.view(np.int32)])
    return {"n_miss": nm, "miss": miss, "state": state, "final": st}


@pytest.mark.parametrize("lib_name", ["product", "reference"])
@pytest.mark.parametrize("policy", [LRU, LFU])
@pytest.mark.parametrize("suite", _suites(), ids=lambda s: s[0])
def test_reference_policy_suites(suite, policy, lib_name):
    name, E, S, ids, md, mi = suite
    h = gu.lib() if lib_name == "product" else gu.ref_lib()
    if h is None:
        pytest.skip("reference library not built")
    hot = sorted(np.random.default_rng(1).choice(E, S, replace=False).tolist())
    decay = 8
    got = gu.run_trace(h, ids.astype(np.int32)[:, None, :], E, S, policy, decay, hot=hot,
                       md=md, mi=mi, gate=False)
    want = _oracle_steps(ids.astype(np.int32), E, S, md, mi, policy, decay, hot)
    _assert_same(got, want, ("n_miss", "miss", "state"), f"{lib_name}:{name}")
    assert np.array_equal(got["final"].routed[0].cpu().numpy(), want["final"].routed)


def _recorded_trace(path) -> np.ndarray:
    """A trace in the replay format (npz "ids" [T, L, mk], -1 padding): the file TRACE names
    if it exists, else one written here through save_routes -- 400 steps x 8 layers of 1 to
    5 tokens x top-10 over 512 experts (Zipf 1.1 with 0.6 per-expert repeat), padded to 50
    ids -- and read back through load_routes."""
    import os
    tr = os.environ.get("TRACE", "routes.npz")
    if os.path.exists(tr):
        return traces.load_routes(tr)
    rng = np.random.default_rng(7)
    E, T, L, K, TOK = 512, 400, 8, 10, 5
    w = np.arange(1, E + 1, dtype=float) ** -1.1
    w /= w.sum()
    ids = np.full((T, L, TOK * K), -1, np.int32)
    for l in range(L):
        perm = rng.permutation(E)
        prev = [perm[rng.choice(E, K, replace=False, p=w)] for _ in range(TOK)]
        for t in range(T):
            for j in range(int(rng.integers(1, TOK + 1))):
                keep = prev[j][rng.random(K) < 0.6]
                fill = [e for e in perm[rng.choice(E, 3 * K, p=w)] if e not in keep]
                row = np.concatenate([keep, np.array(fill[:K - len(keep)], np.int64)])
                ids[t, l, j * K:(j + 1) * K] = row
                prev[j] = row
    traces.save_routes(str(path), ids)
    return traces.load_routes(str(path))


@pytest.mark.parametrize("lib_name", ["product", "reference"])
@pytest.mark.parametrize("policy", [LRU, LFU])
def test_real_trace_suite(tmp_path, policy, lib_name):
    """The reference's sixth policy suite (tests/test_policy.py:222-232) on a trace in its
    replay format: layer TRACE_LAYER (default 7), the first 400 steps, each step's ids with
    the -1 padding removed (so mk varies per step), E = 512, S = 257, max_distinct = 128,
    max_inserts = 64, against the oracle after every step."""
    import os
    h = gu.lib() if lib_name == "product" else gu.ref_lib()
    if h is None:
        pytest.skip("reference library not built")
    ids_all = _recorded_trace(tmp_path / "routes.npz")
    layer = int(os.environ.get("TRACE_LAYER", "7"))
    rows = [ids_all[t, layer][ids_all[t, layer] >= 0].astype(np.int32)
            for t in range(min(400, ids_all.shape[0]))]
    E, S, md, mi, decay = 512, 257, 128, 64, 8
    hot = sorted(np.random.default_rng(1).choice(E, S, replace=False).tolist())
    st = gu.Layers(1, E, S, miss_cap=mi, hot=hot)
    T = len(rows)
    rec = {k: torch.zeros(shape, dtype=torch.int32, device=gu.DEV) for k, shape in (
        ("n_miss", (T, 1)), ("miss", (T, 1, 2 * mi)),
        ("state", (T, 1, oracle.state_words(E, S))))}
    d_rows = [torch.as_tensor(r, device=gu.DEV) for r in rows]
    for t, r in enumerate(d_rows):
        assert gu.manage_call(h, st, 0, gu.ptr(r) if r.numel() else None, r.numel(), md, mi,
                              policy, decay) == 0
        rec["n_miss"][t].copy_(st.n_miss[:, 0])
        rec["miss"][t].copy_(st.miss)
        rec["state"][t].copy_(st.state_words())
    torch.cuda.synchronize()
    got = {k: v.cpu().numpy() for k, v in rec.items()}
    ref = oracle.State(E, S, hot, miss_cap=mi)
    want = {k: np.zeros_like(v) for k, v in got.items()}
    for t, r in enumerate(rows):
        assert ref.manage(r, md, mi, policy, decay) == 0
        want["n_miss"][t, 0] = ref.n_miss[0]
        want["miss"][t, 0] = ref.miss
        want["state"][t, 0] = np.concatenate([ref.table, ref.map_cold, ref.slot_expert,
                                              ref.slot_stamp.view(np.int32),
                                              ref.step.view(np.int32)])
    _assert_same(got, want, ("n_miss", "miss", "state"), f"{lib_name}:real-trace-L{layer}")
    assert int(want["n_miss"].sum()) > 0


REF_CASES = [("48-layer-e128", 16, "lfu", 2048), ("48-layer-e128-batch4", 32, "lfu", 2048),
             ("8-layer-e256-fp8", 128, "lru", 2048)]


@pytest.mark.parametrize("name,slots,policy,steps", REF_CASES)
def test_reference_kernel_agrees_with_oracle(name, slots, policy, steps):
    """The reference's own kernel on the workloads: pins the oracle to the reference."""
    h = gu.ref_lib()
    if h is None:
        pytest.skip("reference library not built")
    w = traces.WORKLOADS[name]
    ids = traces.routing_all_layers(w, steps=min(w.steps, steps))
    got = gu.run_trace(h, ids, w.experts, slots, POLICY[policy])
    want = gu.oracle_trace(ids, w.experts, slots, POLICY[policy])
    _assert_same(got, want, ("n_miss", "miss", "state"), f"reference:{name}")


@pytest.mark.parametrize("policy", ["lfu", "lru"])
def test_product_equals_reference_kernel_over_the_whole_trace(policy):
    """The benchmark workload at its 64-slot budget, all 48 layers x 4096 steps from a cold
    start: the reference's kernel, this library's product entry point (policy step + fused
    remap) and the oracle, compared on every field of every step. The product is compared
    with the reference's kernel directly, not only through the oracle, and its slot ids
    with the reference's table after each step (cache.py:108-110 of the reference)."""
    h = gu.ref_lib()
    if h is None:
        pytest.skip("reference library not built")
    w = traces.WORKLOADS["48-layer-e128"]
    ids = traces.routing_all_layers(w)
    assert ids.shape == (4096, 48, 8)
    ref = gu.run_trace(h, ids, w.experts, 64, POLICY[policy])
    got = gu.run_trace(gu.lib(), ids, w.experts, 64, POLICY[policy], fused_remap=True)
    _assert_same(got, ref, ("n_miss", "miss", "state"), f"product-vs-reference:{policy}")
    _assert_same({"out": got["out"]}, {"out": _expected_remap(ids, ref["state"], w.experts)},
                 ("out",), f"product-vs-reference:{policy}")
    del got
    want = gu.oracle_trace(ids, w.experts, 64, POLICY[policy])
    _assert_same(ref, want, ("n_miss", "miss", "state"), f"reference-vs-oracle:{policy}")
    print(f"whole trace {policy}: {int(want['n_miss'].sum())} inserts over "
          f"{ids.shape[0]} x {ids.shape[1]} layer-steps, identical", flush=True)


def test_deterministic_across_runs():
    w = traces.WORKLOADS["48-layer-e128-batch4"]
    ids = traces.routing_all_layers(w, steps=256)[:, :4]
    a = gu.run_trace(gu.lib(), ids, w.experts, 48, LFU, fused_remap=True)
    b = gu.run_trace(gu.lib(), ids, w.experts, 48, LFU, fused_remap=True)
    for k in ("n_miss", "miss", "state", "out"):
        assert np.array_equal(a[k], b[k]), k


def test_int64_ids_and_padding_through_fused_remap():
    """int64 routing ids (truncated to int32 for the policy, like .to(torch.int32)) and
    padding / out-of-range ids; remap wraps negatives and writes -1 outside [-E, E)."""
    E, S = 128, 32
    rng = np.random.default_rng(9)
    st_dev = gu.Layers(1, E, S)
    st_ref = oracle.State(E, S)
    for t in range(200):
        ids = rng.integers(-3, 130, size=24).astype(np.int64)
        ids[rng.integers(0, 24)] = (1 << 33) + 5  # truncates to 5 for the policy
        d_ids = torch.as_tensor(ids, device=gu.DEV)
        out = torch.empty_like(d_ids)
        rc = gu.manage_call(gu.lib(), st_dev, 0, gu.ptr(d_ids), ids.size, 24, S, LFU, 16,
                            gu.ptr(out), id_bytes=8)
        assert rc == 0
        assert st_ref.manage(ids.astype(np.int32), 24, S, LFU, 16) == 0
        torch.cuda.synchronize()
        assert np.array_equal(st_dev.table[0].cpu().numpy(), st_ref.table)
        assert np.array_equal(st_dev.slot_stamp[0].cpu().numpy(), st_ref.slot_stamp)
        assert np.array_equal(out.cpu().numpy(), oracle.remap(ids, st_ref.table))


@pytest.mark.parametrize("entry", ["manage", "manage_remap", "fused"])
def test_empty_routing(entry):
    """mk = 0 (no routing ids, a null ids pointer): the step counter advances, nothing is
    routed, nothing inserted; the state is otherwise untouched."""
    E, S = 64, 16
    st = gu.Layers(1, E, S, hot=list(range(0, 32, 2)))
    st.slot_stamp.fill_(5)
    before = {f: getattr(st, f).clone() for f in ("table", "map_cold", "slot_expert",
                                                  "slot_stamp")}
    if entry == "fused":
        outs = {k: torch.full((n,), -5, dtype=torch.int32, device=gu.DEV) for k, n in
                (("sorted_hot", 16), ("eids_hot", 1), ("npad_hot", 1), ("sorted_cold", 16),
                 ("eids_cold", 1), ("npad_cold", 1))}
        rc = gu.lib().expert_cache_fused(
            None, 0, E, S, 0, S, st.row("table", 0), st.row("map_cold", 0),
            st.row("slot_expert", 0), st.row("slot_stamp", 0), st.row("routed", 0),
            st.row("step", 0), st.row("miss", 0), st.row("n_miss", 0), 16, 16, 1,
            *[gu.ptr(outs[k]) for k in ("sorted_hot", "eids_hot", "npad_hot", "sorted_cold",
                                        "eids_cold", "npad_cold")], gu.stream())
    elif entry == "manage":
        rc = gu.manage_call(gu.lib(), st, 0, None, 0, 0, S, LFU, 64)
    else:
        out = torch.full((1,), -5, dtype=torch.int32, device=gu.DEV)
        rc = gu.manage_call(gu.lib(), st, 0, None, 0, 0, S, LFU, 64, out_ptr=gu.ptr(out))
    assert rc == 0
    torch.cuda.synchronize()
    assert int(st.step[0, 0]) == 1 and int(st.n_miss[0, 0]) == 0
    assert int(st.routed.sum()) == 0
    for f, t in before.items():
        assert torch.equal(getattr(st, f), t), f
    if entry == "fused":
        assert outs["npad_hot"].item() == 0 and outs["npad_cold"].item() == 0
        assert (outs["sorted_hot"] == 0).all() and (outs["eids_hot"] == -1).all()
