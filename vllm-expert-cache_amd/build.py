"""Build the in-tree libraries of the vllm_expert_cache package.

  libexpertcache.so  gfx950 kernels + C-ABI (csrc/expert_cache.hip), hipcc
  libectrace.so      routing-trace generator (csrc/traces.c), host C

Both land next to the package (vllm_expert_cache/), where _lib.py and traces.py look first.
Every symbol declared in include/expert_cache.h must be exported, or the build fails.

    python vllm-expert-cache_amd/build.py
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
PKG = HERE / "vllm_expert_cache"
HEADER = ROOT / "include" / "expert_cache.h"

ARCH = os.environ.get("EXPERT_CACHE_ARCH", "gfx950")
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
             # keep hipcc from emitting packed-FP32 instructions (v_pk_*_f32)
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.access(c, os.X_OK):
            return c
    raise FileNotFoundError("hipcc not found; set HIPCC")


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^int\s+(expert_cache_\w+)\s*\(", text, re.M)))


def exported_symbols(so: Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(so)], check=True,
                         capture_output=True, text=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that is noise
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msg = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{msg}")
    if msg.strip() and verbose:
        print(msg)


def build_kernels(verbose: bool = False) -> Path:
    out = PKG / "libexpertcache.so"
    tmp = out.with_suffix(".so.tmp")
    _run([hipcc(), *HIP_FLAGS, "-I", str(ROOT / "include"), str(CSRC / "expert_cache.hip"),
          "-o", str(tmp)], verbose)
    missing = [s for s in declared_symbols() if s not in exported_symbols(tmp)]
    if missing:
        tmp.unlink()
        raise RuntimeError(f"libexpertcache.so does not export {missing}")
    os.replace(tmp, out)
    return out


def build_traces(verbose: bool = False) -> Path:
    out = PKG / "libectrace.so"
    cc = os.environ.get("CC", "gcc")
    _run([cc, "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-Wextra",
          str(CSRC / "traces.c"), "-o", str(out), "-lm"], verbose)
    return out


def build(verbose: bool = False) -> None:
    build_kernels(verbose)
    build_traces(verbose)


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
    print("built", PKG / "libexpertcache.so", "and", PKG / "libectrace.so")
