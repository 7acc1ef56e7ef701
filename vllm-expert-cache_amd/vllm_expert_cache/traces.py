"""Routing traces and expert layouts of the expert-cache workloads.

Two sources of routing:
  * synthetic traces from libectrace.so (csrc/traces.c), a pure function of (shape, seed);
  * recorded traces in the reference's replay format, an npz whose "ids" array is
    [T, L, mk] int with -1 padding (tests/test_policy.py:222-232), via `load_routes`.

WORKLOADS names the five shapes the cache is exercised on. Every layer of a workload has
its own seed, seed0 + layer, so layer 0 of the 48-layer workload is the single-layer one.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = Path(__file__).parent / "libectrace.so"
        if not path.is_file():
            raise FileNotFoundError(f"{path} missing: run `python vllm-expert-cache_amd/build.py`")
        h = ctypes.CDLL(str(path))
        h.ectrace_locality.restype = ctypes.c_int
        h.ectrace_locality.argtypes = [ctypes.c_void_p] + [ctypes.c_int] * 4 + \
            [ctypes.c_double, ctypes.c_double, ctypes.c_uint64]
        h.ectrace_grouped.restype = ctypes.c_int
        h.ectrace_grouped.argtypes = [ctypes.c_void_p] + [ctypes.c_int] * 6 + \
            [ctypes.c_double, ctypes.c_uint64]
        _LIB = h
    return _LIB


@dataclass(frozen=True)
class Buffer:
    """One per-expert tensor: name and bytes per expert (shape and dtype for the record)."""
    name: str
    shape: tuple
    dtype: str
    itemsize: int

    @property
    def nbytes(self) -> int:
        return int(np.prod(self.shape)) * self.itemsize


@dataclass(frozen=True)
class Workload:
    name: str
    experts: int
    top_k: int
    tokens: int
    layers: int
    steps: int
    slots: tuple
    buffers: tuple
    routing: str            # "locality" or "grouped"
    zipf_s: float = 1.1
    keep: float = 0.6
    groups: int = 0
    topk_groups: int = 0
    seed0: int = 0
    policies: tuple = ("lfu", "lru")
    extra: dict = field(default_factory=dict)

    @property
    def mk(self) -> int:
        return self.tokens * self.top_k

    @property
    def bytes_per_expert(self) -> int:
        return sum(b.nbytes for b in self.buffers)


# W8A8 int8 experts with fp32 per-channel scales: w13 [1536, 2048], w2 [2048, 768]
_W8A8 = (Buffer("w13_weight", (1536, 2048), "int8", 1),
         Buffer("w2_weight", (2048, 768), "int8", 1),
         Buffer("w13_weight_scale", (1536, 1), "float32", 4),
         Buffer("w2_weight_scale", (2048, 1), "float32", 4))
# Mixtral-sized bf16 experts: w13 [28672, 4096], w2 [4096, 14336]
_BF16_BIG = (Buffer("w13_weight", (28672, 4096), "bfloat16", 2),
             Buffer("w2_weight", (4096, 14336), "bfloat16", 2))
# DeepSeek-V3-sized fp8 e4m3 experts with 128x128 fp32 block scales
_FP8_BLOCK = (Buffer("w13_weight", (4096, 7168), "float8_e4m3fn", 1),
              Buffer("w2_weight", (7168, 2048), "float8_e4m3fn", 1),
              Buffer("w13_weight_scale_inv", (32, 56), "float32", 4),
              Buffer("w2_weight_scale_inv", (56, 16), "float32", 4))

WORKLOADS = {
    # single MoE layer: 128 experts, top-8, 64 slots, 1 token/step, 4096 steps
    "single-layer-e128": Workload("single-layer-e128", 128, 8, 1, 1, 4096, (64,), _W8A8,
                                  "locality", seed0=1000),
    # 48 such layers, one seed each, slot budgets 16..96
    "48-layer-e128": Workload("48-layer-e128", 128, 8, 1, 48, 4096, (16, 32, 48, 64, 96),
                              _W8A8, "locality", seed0=1000),
    # batched decode: 4 tokens/step (32 ids), budgets on both sides of 32
    "48-layer-e128-batch4": Workload("48-layer-e128-batch4", 128, 8, 4, 48, 2048,
                                     (24, 32, 48), _W8A8, "locality", seed0=2000),
    # few large experts: 8 bf16 experts of 352 MB, top-2, 4 slots, uniform routing with a
    # per-expert repeat probability of 0.5
    "8-layer-e8-bf16": Workload("8-layer-e8-bf16", 8, 2, 1, 8, 256, (4,), _BF16_BIG,
                                "locality", zipf_s=0.0, keep=0.5, seed0=3000),
    # many experts: 256 fp8 experts, top-8, 16 tokens/step, group-limited routing
    "8-layer-e256-fp8": Workload("8-layer-e256-fp8", 256, 8, 16, 8, 1024, (128,), _FP8_BLOCK,
                                 "grouped", groups=8, topk_groups=4, seed0=4000),
}


def routing(w: Workload, layer: int = 0, steps: int | None = None) -> np.ndarray:
    """Routing ids [steps, tokens * top_k] int32 of one layer of workload `w`."""
    T = w.steps if steps is None else int(steps)
    out = np.empty((T, w.mk), dtype=np.int32)
    seed = ctypes.c_uint64(w.seed0 + layer)
    if w.routing == "locality":
        rc = _lib().ectrace_locality(out.ctypes.data, T, w.tokens, w.top_k, w.experts,
                                     w.zipf_s, w.keep, seed)
    else:
        rc = _lib().ectrace_grouped(out.ctypes.data, T, w.tokens, w.top_k, w.experts,
                                    w.groups, w.topk_groups, w.zipf_s, seed)
    if rc != 0:
        raise ValueError(f"trace generator rejected {w.name} (rc={rc})")
    return out


def routing_all_layers(w: Workload, steps: int | None = None) -> np.ndarray:
    """[steps, layers, mk] int32."""
    return np.stack([routing(w, layer, steps) for layer in range(w.layers)], axis=1)


def load_routes(path: str) -> np.ndarray:
    """A recorded trace in the reference's replay format: npz with "ids" [T, L, mk], -1
    padding. Loaded without unpickling."""
    with np.load(path, allow_pickle=False) as d:
        ids = np.asarray(d["ids"])
    if ids.ndim != 3:
        raise ValueError(f"expected ids[T, L, mk], got shape {ids.shape}")
    return ids.astype(np.int32)


def save_routes(path: str, ids: np.ndarray) -> None:
    np.savez(path, ids=np.asarray(ids, dtype=np.int32))


# ---- synthetic expert content ------------------------------------------------------------
# Every 4-byte word of a synthetic expert slab is a hash of its position: (layer, expert,
# buffer, word). A copy that lands in the wrong slot, takes another expert's or layer's row,
# or shifts any 16-byte vector within a slab therefore shows up as a mismatch, which random
# or constant bytes would not guarantee.

_M32 = 0xFFFFFFFF
_MUL = 0x045D9F3B  # odd: multiplication by it is a bijection mod 2**32


def _mix32(x):
    """A bijective 32-bit mixer (xor-shift, odd multiply, twice, then xor-shift) on int64
    tensors holding values below 2**32: every product stays below 2**59."""
    x = ((x ^ (x >> 16)) * _MUL) & _M32
    x = ((x ^ (x >> 16)) * _MUL) & _M32
    return x ^ (x >> 16)


def expert_words(layer: int, experts, buffer: int, nbytes: int, device, first_word: int = 0,
                 nwords: int | None = None):
    """Synthetic content of `buffer`'s slab for each expert in `experts` of `layer`, as
    int32 words [len(experts), nwords] (words first_word .. of a slab of nbytes, which must
    be a multiple of 4). Requires layer < 2048, buffer < 16, expert ids in [0, 65536)."""
    import torch

    if nbytes % 4 or not (0 <= layer < 2048 and 0 <= buffer < 16):
        raise ValueError("expert_words: nbytes % 4, layer or buffer out of range")
    n = nbytes // 4 - first_word if nwords is None else int(nwords)
    e = torch.as_tensor(experts, dtype=torch.int64, device=device).reshape(-1, 1)
    if e.numel() and (int(e.min()) < 0 or int(e.max()) >= 65536):
        raise ValueError("expert_words: expert id out of range")
    seed = _mix32((layer << 20) ^ (buffer << 16) ^ e)
    w = torch.arange(first_word, first_word + n, dtype=torch.int64, device=device).reshape(1, -1)
    h = _mix32(w ^ seed)
    h = _mix32((h + seed) & _M32)
    return h.to(torch.int32)


def fill_expert_store(host, layer: int, buffer: int, nbytes: int, experts: int, device,
                      chunk_words: int = 1 << 26) -> None:
    """Write expert_words of experts 0..experts-1 into `host` (a [experts * nbytes] uint8
    tensor, pinned or on the device), generated on `device` in chunks of at most
    chunk_words words."""
    import torch

    view = host.view(torch.int32).view(experts, nbytes // 4)
    per = nbytes // 4
    if per <= chunk_words:
        step = max(1, chunk_words // per)
        for e0 in range(0, experts, step):
            e1 = min(experts, e0 + step)
            view[e0:e1].copy_(expert_words(layer, range(e0, e1), buffer, nbytes, device))
    else:
        for e in range(experts):
            for w0 in range(0, per, chunk_words):
                n = min(chunk_words, per - w0)
                view[e, w0:w0 + n].copy_(expert_words(layer, [e], buffer, nbytes, device,
                                                      w0, n)[0])


def slots_match(slot_buf, slot_expert, layer: int, buffer: int, nbytes: int,
                chunk_words: int = 1 << 26) -> tuple[bool, int]:
    """Does every resident slot of `slot_buf` ([S * nbytes] uint8 on the device) hold its
    expert's expert_words? slot_expert: [S] int32 tensor (-1 for an empty slot). Returns
    (all equal, slots compared)."""
    import torch

    per = nbytes // 4
    view = slot_buf.view(torch.int32).view(-1, per)
    se = slot_expert.to(torch.int64)
    resident = torch.nonzero(se >= 0).flatten()
    experts = se[resident]
    ok = True
    if per <= chunk_words:
        step = max(1, chunk_words // per)
        for i in range(0, resident.numel(), step):
            want = expert_words(layer, experts[i:i + step], buffer, nbytes, slot_buf.device)
            ok = ok and bool(torch.equal(view[resident[i:i + step]], want))
    else:
        for s, e in zip(resident.tolist(), experts.tolist()):
            for w0 in range(0, per, chunk_words):
                n = min(chunk_words, per - w0)
                want = expert_words(layer, [e], buffer, nbytes, slot_buf.device, w0, n)[0]
                ok = ok and bool(torch.equal(view[s, w0:w0 + n], want))
    return ok, int(resident.numel())
