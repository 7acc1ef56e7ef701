"""Environment semantics of vllm_expert_cache.config (reference config.py:8-47)."""
from __future__ import annotations

import logging

import pytest

import vllm_expert_cache
from vllm_expert_cache.config import settings


@pytest.fixture(autouse=True)
def _clean(monkeypatch):
    for k in ("EXPERT_CACHE_DISABLE", "EXPERT_CACHE_SLOTS", "EXPERT_CACHE_FRACTION",
              "EXPERT_CACHE_POLICY", "EXPERT_CACHE_DECAY"):
        monkeypatch.delenv(k, raising=False)


def test_defaults():
    assert settings.disabled is False
    assert settings.slots is None
    assert settings.fraction == 0.5
    assert settings.policy == "lfu" and settings.policy_code == 1
    assert settings.decay == 64
    assert vllm_expert_cache.__version__ == "0.2.0"


def test_policy_parsing(monkeypatch):
    for raw, code in ((" LRU ", 0), ("lfu", 1), ("LfU", 1), ("arc", 0), ("", 0)):
        monkeypatch.setenv("EXPERT_CACHE_POLICY", raw)
        assert settings.policy_code == code, raw


def test_slots_for(monkeypatch):
    assert settings.slots_for(128) == 64
    monkeypatch.setenv("EXPERT_CACHE_FRACTION", "0.25")
    assert settings.slots_for(10) == 2        # round(2.5) is 2: half to even
    assert settings.slots_for(14) == 4        # round(3.5) is 4
    monkeypatch.setenv("EXPERT_CACHE_FRACTION", "0.0")
    assert settings.slots_for(128) == 1       # at least one slot
    monkeypatch.setenv("EXPERT_CACHE_SLOTS", "500")
    assert settings.slots_for(128) == 128     # at most E
    monkeypatch.setenv("EXPERT_CACHE_SLOTS", "")
    assert settings.slots is None


def test_live_reads(monkeypatch):
    monkeypatch.setenv("EXPERT_CACHE_DISABLE", "1")
    assert settings.disabled
    monkeypatch.setenv("EXPERT_CACHE_DISABLE", "true")  # only "1" disables
    assert not settings.disabled
    monkeypatch.setenv("EXPERT_CACHE_DECAY", "0")
    assert settings.decay == 0


def test_install_honours_disable(monkeypatch, caplog):
    monkeypatch.setenv("EXPERT_CACHE_DISABLE", "1")
    with caplog.at_level(logging.INFO, logger="vllm.expert_cache"):
        vllm_expert_cache.install()
    assert "disabled by EXPERT_CACHE_DISABLE" in caplog.text


def test_entry_point_text():
    from pathlib import Path

    text = (Path(vllm_expert_cache.__file__).parent.parent / "pyproject.toml").read_text()
    assert '[project.entry-points."vllm.general_plugins"]' in text
    assert 'expert_cache = "vllm_expert_cache:install"' in text


def test_gather_grids_from_the_environment(monkeypatch):
    """The gather grid (EXPERT_CACHE_CHUNKS / _LANES, as in the reference) and the prefetch
    copy grid (EXPERT_CACHE_PREFETCH_CHUNKS) are read when a cache is built; the defaults
    are 32 x 1 and 16."""
    import torch

    from vllm_expert_cache.cache import ExpertSlotCache

    owner = torch.nn.Module()
    owner.w = torch.nn.Parameter(torch.zeros(8, 4), requires_grad=False)
    for k in ("EXPERT_CACHE_CHUNKS", "EXPERT_CACHE_LANES", "EXPERT_CACHE_PREFETCH_CHUNKS"):
        monkeypatch.delenv(k, raising=False)
    c = ExpertSlotCache(owner, ["w"], 8, 2, "cpu")
    assert (c.chunks, c.lanes, c.pf_chunks) == (32, 1, 16)
    monkeypatch.setenv("EXPERT_CACHE_CHUNKS", "16")
    monkeypatch.setenv("EXPERT_CACHE_LANES", "64")
    monkeypatch.setenv("EXPERT_CACHE_PREFETCH_CHUNKS", "8")
    c = ExpertSlotCache(owner, ["w"], 8, 2, "cpu")
    assert (c.chunks, c.lanes, c.pf_chunks) == (16, 64, 8)
