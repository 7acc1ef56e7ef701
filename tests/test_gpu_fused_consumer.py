"""expert_cache_fused's outputs as the downstream MoE consumes them.

The fused entry point hands vLLM's block-sparse expert GEMM two moe_align_block_size
layouts (kernels/expert_cache.hip:431-588): the resident ids bucketed by slot (their rows
are read from the HBM slot buffers) and the rest bucketed by expert id (read through from
the full host tensors). Each block of `bs` rows belongs to one slot or expert, and each row
is an index into the step's flattened topk ids, with `mk` as padding.

Here a block-sparse MoE written in torch consumes exactly those outputs -- per block, the
rows' tokens times that block's weight matrix, scattered back with the routing weights --
and must equal the dense MoE over the same routing, step after step. A small insert cap
keeps some routed experts non-resident, so both sides carry rows. Every routed position
must appear exactly once across the two sides.
"""
from __future__ import annotations

import numpy as np
import torch

import pytest

import gpu_util as gu
from test_oracle import align_lengths

pytestmark = pytest.mark.gpu

E, S, K, TOK, H, N, BS = 128, 32, 8, 4, 32, 16, 16


def _block_moe(x, wts, sorted_ids, eids, npad, weights, mk):
    """The consumer: blocks [0, npad / bs) of one side, block b using weights[eids[b]]."""
    nblk = int(npad) // BS
    if nblk == 0:
        return torch.zeros(x.shape[0], N, device=x.device), torch.zeros(0, dtype=torch.long)
    e = eids[:nblk].long()
    rows = sorted_ids[:nblk * BS].view(nblk, BS).long()
    use = (rows < mk) & (e >= 0)[:, None]
    r = torch.where(use, rows, torch.zeros_like(rows))
    tok = r // K
    xs = x[tok]                                                   # [nblk, BS, H]
    wb = weights[e.clamp(min=0)].contiguous()                     # [nblk, H, N]
    y = torch.bmm(xs, wb) * (wts.flatten()[r] * use)[..., None]   # [nblk, BS, N]
    out = torch.zeros(x.shape[0], N, device=x.device)
    out.index_add_(0, tok.flatten(), y.reshape(-1, N))
    return out, rows[use].cpu()


def test_block_sparse_moe_from_fused_outputs_equals_dense():
    h = gu.lib()
    mk = TOK * K
    L, NB = align_lengths(mk, E, BS)
    g = torch.Generator(device=gu.DEV).manual_seed(4)
    W = torch.randn(E, H, N, device=gu.DEV, generator=g)          # full expert weights
    st = gu.Layers(1, E, S, miss_cap=S)
    outs = {k: torch.full((n,), -5, dtype=torch.int32, device=gu.DEV) for k, n in
            (("sorted_hot", L), ("eids_hot", NB), ("npad_hot", 1),
             ("sorted_cold", L), ("eids_cold", NB), ("npad_cold", 1))}
    rng = np.random.default_rng(9)
    cold_rows = 0
    for t in range(40):
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(TOK)]).astype(np.int32)
        d_ids = torch.as_tensor(ids, device=gu.DEV)
        x = torch.randn(TOK, H, device=gu.DEV, generator=g)
        wts = torch.softmax(torch.randn(TOK, K, device=gu.DEV, generator=g), dim=-1)
        cap = 2 if t % 3 else S  # a small insert cap leaves routed experts non-resident
        rc = h.expert_cache_fused(
            gu.ptr(d_ids), mk, E, S, E, cap, st.row("table", 0), st.row("map_cold", 0),
            st.row("slot_expert", 0), st.row("slot_stamp", 0), st.row("routed", 0),
            st.row("step", 0), st.row("miss", 0), st.row("n_miss", 0), BS, L, NB,
            *[gu.ptr(outs[k]) for k in ("sorted_hot", "eids_hot", "npad_hot", "sorted_cold",
                                        "eids_cold", "npad_cold")], gu.stream())
        assert rc == 0
        # the gather's effect: every resident slot holds its expert's weights
        se = st.slot_expert[0].long()
        W_slot = W[se.clamp(min=0)]
        hot, rows_h = _block_moe(x, wts, outs["sorted_hot"], outs["eids_hot"],
                                 outs["npad_hot"][0], W_slot, mk)
        cold, rows_c = _block_moe(x, wts, outs["sorted_cold"], outs["eids_cold"],
                                  outs["npad_cold"][0], W, mk)
        d = d_ids.long()
        per = torch.bmm(x[:, None, :].expand(TOK, K, H).reshape(-1, 1, H).contiguous(),
                        W[d.flatten()].contiguous()).view(TOK, K, N)
        dense = (per * wts[..., None]).sum(1)
        torch.cuda.synchronize()
        assert torch.allclose(hot + cold, dense, rtol=1e-5, atol=1e-5), \
            f"step {t}: max |diff| {float((hot + cold - dense).abs().max())}"
        placed = np.sort(np.concatenate([rows_h.numpy(), rows_c.numpy()]))
        assert np.array_equal(placed, np.arange(mk)), t  # each position exactly once
        cold_rows += len(rows_c)
    assert cold_rows > 0  # the cold side was exercised
