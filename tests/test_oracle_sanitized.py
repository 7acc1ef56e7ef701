"""The oracle's C (oracle/policy.c) under AddressSanitizer and UndefinedBehaviorSanitizer.

oracle/selftest.c drives random shapes through every oracle entry point -- the policy step
under both victim rules (compared after every step, invariants checked), prefetch, the
fused step and remap -- including E = 1, S > E, no ids, padding and out-of-range ids,
insert caps from 0 to 1024 and stamps at the limits of int64. Built and run through
`make -C oracle selftest` into a temporary directory; any sanitizer report or rule
mismatch fails the test.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ORACLE = Path(__file__).resolve().parents[1] / "oracle"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_oracle_runs_clean_under_sanitizers(tmp_path):
    out = tmp_path / "selftest"
    r = subprocess.run(["make", "-s", "-C", str(ORACLE), "selftest", f"SELFTEST={out}",
                        "CASES=400"], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert "400 cases passed" in r.stdout
