"""The oracle against vectors written by the reference's own policy kernel.

tests/golden/reference_policy_suites.npz holds what kernels/expert_cache.hip, compiled
unchanged, produced on a GPU over the routing of the reference's five policy suites under
both policies (tests/golden/make_reference_vectors.py made it). Each step's n_miss, whole
miss buffer and state digest, and each run's final state, must come out of the oracle
exactly, under both of its victim rules. No GPU and no reference tree are needed here.
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
SUITES = sorted({k.split("/")[0] for k in DATA if not k.startswith("meta/")})


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
