"""The oracle against vectors written by the reference's own policy kernel.

tests/golden/reference_policy_suites.npz holds what kernels/expert_cache.hip, compiled
unchanged, produced on a GPU (tests/golden/make_reference_vectors.py made it):
  * its policy kernel over the routing of the reference's five policy suites under both
    policies: each step's n_miss, whole miss buffer and state digest, and each run's final
    state, must come out of the oracle exactly, under both of its victim rules;
  * its fused kernel over four workloads (block sizes 16 and 3, padding and out-of-range
    ids included): each step's digest of both align outputs and the state, and the last
    step's outputs, must come out of the oracle's fused step exactly.
No GPU and no reference tree are needed here.
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import pytest

from oracle import State

FIXTURE = Path(__file__).parent / "golden" / "reference_policy_suites.npz"


def _load():
    with np.load(FIXTURE, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


DATA = _load()
SUITES = sorted({k.split("/")[0] for k in DATA if k.endswith("/p0/digest")})
FUSED = sorted({k.split("/")[0] for k in DATA if k.startswith("fused-")})
FUSED_KEYS = ("sorted_hot", "eids_hot", "npad_hot", "sorted_cold", "eids_cold", "npad_cold")


def _words(s: State) -> np.ndarray:
    return np.concatenate([s.table, s.map_cold, s.slot_expert, s.slot_stamp.view(np.int32),
                           s.step.view(np.int32)]).astype(np.int32)


def test_fixture_covers_the_five_suites_and_both_policies():
    assert SUITES == ["insert-capped", "padded-rows", "read-through", "skewed-512",
                      "tiny-churn"]
    for name in SUITES:
        for policy in (0, 1):
            assert f"{name}/p{policy}/digest" in DATA
    inserts = sum(int(DATA[f"{n}/p{p}/n_miss"].sum()) for n in SUITES for p in (0, 1))
    assert inserts > 5000


@pytest.mark.parametrize("rule", ["rank", "serial"])
@pytest.mark.parametrize("policy", [0, 1])
@pytest.mark.parametrize("name", SUITES)
def test_oracle_reproduces_the_reference_kernel(name, policy, rule):
    E, S, md, mi = (int(x) for x in DATA[f"{name}/shape"])
    ids = DATA[f"{name}/ids"].astype(np.int32)
    decay = int(DATA["meta/decay"][0])
    key = f"{name}/p{policy}"
    st = State(E, S, DATA[f"{name}/hot"].tolist(), miss_cap=mi)
    for t in range(ids.shape[0]):
        assert st.manage(ids[t], md, mi, policy, decay, rule) == 0
        assert st.n_miss[0] == DATA[f"{key}/n_miss"][t], (key, t)
        assert np.array_equal(st.miss.astype(np.int16), DATA[f"{key}/miss"][t]), (key, t)
        digest = np.frombuffer(hashlib.sha256(_words(st).tobytes()).digest(), np.uint8)
        assert np.array_equal(digest, DATA[f"{key}/digest"][t]), (key, t)
    assert np.array_equal(_words(st), DATA[f"{key}/final"]), key


def test_fixture_covers_the_fused_workloads():
    assert FUSED == ["fused-48-layer-e128", "fused-48-layer-e128-batch4",
                     "fused-8-layer-e256-fp8", "fused-small-bs3"]


@pytest.mark.parametrize("name", FUSED)
def test_oracle_fused_reproduces_the_reference_kernel(name):
    E, S, bs, L, NB = (int(x) for x in DATA[f"{name}/shape"])
    ids = DATA[f"{name}/ids"].astype(np.int32)
    st = State(E, S)
    mk = ids.shape[1]
    for t in range(ids.shape[0]):
        rc, out = st.fused(ids[t], min(E, mk), S, bs, L, NB)
        assert rc == 0
        assert st.n_miss[0] == DATA[f"{name}/n_miss"][t], (name, t)
        blob = np.concatenate([out[k] for k in FUSED_KEYS] + [_words(st)]).astype(np.int32)
        digest = np.frombuffer(hashlib.sha256(blob.tobytes()).digest(), np.uint8)
        if not np.array_equal(digest, DATA[f"{name}/digest"][t]):
            if t == ids.shape[0] - 1:
                for k in FUSED_KEYS:
                    assert np.array_equal(out[k], DATA[f"{name}/last/{k}"]), (name, k)
            raise AssertionError(f"{name}: step {t} differs from the reference kernel")
    for k in FUSED_KEYS:
        assert np.array_equal(out[k], DATA[f"{name}/last/{k}"]), (name, k)
    assert np.array_equal(_words(st), DATA[f"{name}/final"]), name
