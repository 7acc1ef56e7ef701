"""C-ABI of libexpertcache.so, checked without a GPU.

The library loads here (libamdhip64 loads without a device), exports every entry point
include/expert_cache.h declares, and rejects bad arguments with -1 before any HIP call --
with the same verdicts as the reference library compiled from its own source
(kernels/expert_cache.hip:592-643) where that is built.
"""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

import pytest

import oracle
from vllm_expert_cache import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "expert_cache.h"
P = ctypes.c_void_p


def _declared():
    return sorted(set(re.findall(r"^int\s+(expert_cache_\w+)\s*\(", HEADER.read_text(), re.M)))


@pytest.fixture(scope="module")
def lib():
    return _lib.lib()


@pytest.fixture(scope="module")
def ref():
    if not os.path.isfile(oracle.REF_LIB_PATH):
        pytest.skip("reference library not built (oracle/_ref)")
    return ctypes.CDLL(oracle.REF_LIB_PATH)


def test_exports_every_declared_symbol(lib):
    declared = _declared()
    assert set(declared) == set(_lib.SIGNATURES)
    for name in declared:
        assert hasattr(lib, name), name


_C_CALLER = r"""
#include <stdio.h>
#include "expert_cache.h"

int main(void) {
  int bad = 0;
  /* E = 0, S = 0, a null n_miss, chunks = 0, L = 0: each is refused before any HIP call */
  bad += expert_cache_manage(0, 1, 0, 4, 1, 4, 0, 0, 0, 0, 0, 0, 0, 0, 1, 64, 0) != -1;
  bad += expert_cache_manage_remap(0, 4, 1, 8, 0, 1, 4, 0, 0, 0, 0, 0, 0, 0, 0, 1, 64, 0, 0)
         != -1;
  bad += expert_cache_gather((void*)1, (const void*)1, 16, (void*)1, (const void*)1, 16,
                             (void*)1, (const void*)1, 16, (void*)1, (const void*)1, 16,
                             (void*)1, (const void*)1, 16, (void*)1, (const void*)1, 16,
                             (const int*)1, 0, 32, 1, 0) != -1;
  bad += expert_cache_gather_live((void*)1, (const void*)1, 16, (void*)1, (const void*)1, 16,
                                  (void*)1, (const void*)1, 16, (void*)1, (const void*)1, 16,
                                  (void*)1, (const void*)1, 16, (void*)1, (const void*)1, 16,
                                  (const int*)1, (const int*)1, (const int*)1, 0, 1, 0) != -1;
  bad += expert_cache_fused(0, 1, 8, 4, 1, 4, 0, 0, 0, 0, 0, 0, 0, 0, 16, 0, 1, 0, 0, 0, 0, 0,
                            0, 0) != -1;
  bad += expert_cache_remap(0, 1, 3, 0, 8, 0, 0) != -1;
  bad += expert_cache_prefetch(0, 1, 0, 4, 4, 0, 0, 0, 0, 0, 0, 0, 0) != -1;
  printf("%d\n", bad);
  return bad;
}
"""


def test_header_compiles_as_c_and_links(tmp_path):
    """A plain C11 caller (gcc, no HIP headers) compiles against include/expert_cache.h with
    every warning an error, links against the library, and gets -1 from each refused call."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    src = tmp_path / "caller.c"
    src.write_text(_C_CALLER)
    so = Path(_lib.library_path())
    exe = tmp_path / "caller"
    subprocess.run([gcc, "-std=c11", "-Wall", "-Wextra", "-Werror", f"-I{HEADER.parent}",
                    str(src), "-o", str(exe), f"-L{so.parent}", f"-l:{so.name}",
                    f"-Wl,-rpath,{so.parent}"], check=True, capture_output=True, text=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip() == "0"


def test_library_path_order(tmp_path, monkeypatch):
    fake = tmp_path / "libexpertcache.so"
    fake.write_bytes(b"")
    monkeypatch.setenv("EXPERT_CACHE_LIB", str(fake))
    assert _lib.library_path() == str(fake)
    monkeypatch.setenv("EXPERT_CACHE_LIB", str(tmp_path / "missing.so"))
    assert _lib.library_path().endswith("vllm_expert_cache/libexpertcache.so")


def test_bind_refuses_a_library_without_the_remap(ref):
    with pytest.raises(RuntimeError, match="expert_cache_remap"):
        _lib.bind(ref)


def _manage(h, E, S, mi, pol, name="expert_cache_manage"):
    fn = getattr(h, name)
    fn.restype = ctypes.c_int
    fn.argtypes = _lib.SIGNATURES["expert_cache_manage"]
    return fn(P(1), 1, E, S, 1, mi, P(1), P(1), P(1), P(1), P(1), P(1), P(1), P(1), pol, 64,
              None)


BAD_MANAGE = [(0, 4, 4, 0), (-3, 4, 4, 0), (8, 0, 4, 0), (8, 1025, 4, 0), (8, 4, -1, 0),
              (8, 4, 1025, 0), (8, 4, 4, 2), (8, 4, 4, -1)]


@pytest.mark.parametrize("args", BAD_MANAGE)
def test_manage_rejects(lib, args):
    assert _manage(lib, *args) == -1


@pytest.mark.parametrize("args", BAD_MANAGE)
def test_manage_rejects_like_reference(lib, ref, args):
    assert _manage(lib, *args) == _manage(ref, *args) == -1


def _gather(h, sizes, chunks=16, lanes=64):
    fn = h.expert_cache_gather
    fn.restype = ctypes.c_int
    fn.argtypes = _lib.SIGNATURES["expert_cache_gather"]
    args = []
    for b in sizes:
        args += [P(1), P(1), ctypes.c_long(b)]
    return fn(*args, P(1), P(1), chunks, lanes, None)


BAD_GATHER = [([16, 16, 16, 16, 16, 0], 16, 64), ([16, 16, 16, 16, 8, 16], 16, 64),
              ([-16, 16, 16, 16, 16, 16], 16, 64), ([17, 16, 16, 16, 16, 16], 16, 64),
              ([16] * 6, 0, 64), ([16] * 6, 16, 0), ([16] * 6, -1, 64)]


@pytest.mark.parametrize("sizes,chunks,lanes", BAD_GATHER)
def test_gather_rejects_like_reference(lib, ref, sizes, chunks, lanes):
    assert _gather(lib, sizes, chunks, lanes) == -1
    assert _gather(ref, sizes, chunks, lanes) == -1


@pytest.mark.parametrize("sizes,chunks,lanes", BAD_GATHER)
def test_gather_live_rejects_what_gather_rejects(lib, sizes, chunks, lanes):
    args = []
    for b in sizes:
        args += [P(1), P(1), ctypes.c_long(b)]
    assert lib.expert_cache_gather_live(*args, P(1), P(1), P(1), chunks, lanes, None) == -1


def test_gather_live_rejects_a_null_slot_table(lib):
    args = [P(1), P(1), ctypes.c_long(16)] * 6
    assert lib.expert_cache_gather_live(*args, P(1), P(1), None, 32, 1, None) == -1


def test_gathers_reject_a_null_miss_count(lib):
    # every launch reads *n_miss on the device; a null count is refused before any HIP call
    args = [P(1), P(1), ctypes.c_long(16)] * 6
    assert lib.expert_cache_gather(*args, P(1), None, 32, 1, None) == -1
    assert lib.expert_cache_gather_live(*args, P(1), None, P(1), 32, 1, None) == -1


def _fused(h, E, S, mi, bs, L, NB, mk=1):
    fn = h.expert_cache_fused
    fn.restype = ctypes.c_int
    fn.argtypes = _lib.SIGNATURES["expert_cache_fused"]
    return fn(P(1), mk, E, S, 1, mi, *([P(1)] * 8), bs, L, NB, *([P(1)] * 6), None)


BAD_FUSED = [(0, 4, 4, 16, 16, 1), (1025, 4, 4, 16, 16, 1), (8, 0, 4, 16, 16, 1),
             (8, 1025, 4, 16, 16, 1), (8, 4, -1, 16, 16, 1), (8, 4, 1025, 16, 16, 1),
             (8, 4, 4, 0, 16, 1), (8, 4, 4, 16, 0, 1), (8, 4, 4, 16, 16, 0)]


@pytest.mark.parametrize("args", BAD_FUSED)
def test_fused_rejects_like_reference(lib, ref, args):
    assert _fused(lib, *args) == -1
    assert _fused(ref, *args) == -1
    assert _fused(lib, 8, 4, 4, 16, 16, 1, mk=-1) == _fused(ref, 8, 4, 4, 16, 16, 1, mk=-1)


def test_manage_remap_rejects(lib):
    fn = lib.expert_cache_manage_remap
    base = dict(id_bytes=4, E=8, S=4, mi=4, pol=0)
    for k, v in (("id_bytes", 2), ("id_bytes", 16), ("E", 0), ("S", 0), ("S", 1025),
                 ("mi", -1), ("mi", 1025), ("pol", 3)):
        a = dict(base, **{k: v})
        assert fn(P(1), a["id_bytes"], 1, a["E"], a["S"], 1, a["mi"], *([P(1)] * 8), a["pol"],
                  64, P(1), None) == -1, (k, v)
    # ids to remap but nowhere to put them
    assert fn(P(1), 4, 1, 8, 4, 1, 4, *([P(1)] * 8), 0, 64, None, None) == -1


def test_remap_rejects_and_empty_is_a_no_op(lib):
    fn = lib.expert_cache_remap
    assert fn(P(1), 4, 4, P(1), 0, P(1), None) == -1   # E <= 0
    assert fn(P(1), -1, 4, P(1), 8, P(1), None) == -1  # n < 0
    assert fn(P(1), 4, 3, P(1), 8, P(1), None) == -1   # id_bytes not 4 or 8
    assert fn(None, 0, 4, P(1), 8, None, None) == 0    # nothing to do, no launch


def test_prefetch_rejects(lib):
    """expert_cache_prefetch checks its arguments on the host, before any HIP call."""
    fn = lib.expert_cache_prefetch
    for E, S, mi, mk in ((0, 4, 4, 1), (-1, 4, 4, 1), (8, 0, 4, 1), (8, 1025, 4, 1),
                         (8, 4, -1, 1), (8, 4, 1025, 1), (8, 4, 4, -1)):
        assert fn(P(1), mk, E, S, mi, *([P(1)] * 7), None) == -1, (E, S, mi, mk)


def _manage_prefetch(h, **over):
    """expert_cache_manage_remap_prefetch with E=8, S=4 and every array at its own address
    (never dereferenced: each call below is rejected on the host)."""
    a = {k: 0x100000 + i * 0x1000 for i, k in enumerate(
        ("table", "map_cold", "slot_expert", "slot_stamp", "routed", "miss", "n_miss"))}
    p = {k: 0x200000 + i * 0x1000 for i, k in enumerate(
        ("table", "map_cold", "slot_expert", "slot_stamp", "routed", "miss", "n_miss"))}
    v = dict(id_bytes=4, mk=1, E=8, S=4, md=1, mi=4, policy=1, out=0x300000, pk=1, pmi=4)
    for k, x in over.items():
        if k.startswith("a_"):
            a[k[2:]] = x
        elif k.startswith("p_"):
            p[k[2:]] = x
        else:
            v[k] = x
    return h.expert_cache_manage_remap_prefetch(
        P(0x400000), v["id_bytes"], v["mk"], v["E"], v["S"], v["md"], v["mi"],
        P(a["table"]), P(a["map_cold"]), P(a["slot_expert"]), P(a["slot_stamp"]),
        P(a["routed"]), P(0x500000), P(a["miss"]), P(a["n_miss"]), v["policy"], 64,
        P(v["out"]), P(0x600000), v["pk"], v["pmi"], P(p["table"]), P(p["map_cold"]),
        P(p["slot_expert"]), P(p["slot_stamp"]), P(p["routed"]), P(p["miss"]),
        P(p["n_miss"]), None)


@pytest.mark.parametrize("over", [
    dict(E=0), dict(S=0), dict(S=1025), dict(mi=-1), dict(mi=1025), dict(policy=2),
    dict(id_bytes=2), dict(out=0), dict(pmi=-1), dict(pmi=1025), dict(pk=-1),
    # the two layers' arrays meet: same array, or a range that reaches into the other
    dict(p_table=0x100000), dict(p_map_cold=0x101000 + 28), dict(p_slot_expert=0x102000 - 12),
    dict(p_slot_stamp=0x103000 + 24), dict(p_routed=0x104000 + 7), dict(p_miss=0x105000 + 28),
    dict(p_miss=0x105000 - 28, pmi=4), dict(p_n_miss=0x106000),
], ids=lambda d: ",".join(f"{k}={v}" for k, v in d.items()))
def test_manage_remap_prefetch_rejects(lib, over):
    """expert_cache_manage_remap_prefetch checks its arguments, and that the two layers'
    arrays are disjoint, on the host before any HIP call."""
    assert _manage_prefetch(lib, **over) == -1
