"""GPU parity of the permutation (counting sort) against the CPU oracle:
counts, offsets, row_src (perm), slot (inverse perm) and the GEMM tile
prefixes must be bit-exact, including empty experts, sentinel ids, ragged
S and the 1792-expert bank."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from moe_amd import ops
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _routing(T, E, K, seed, skew=0.0, sentinel_every=0):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=g)
    if skew:
        rank = torch.randperm(E, generator=g).float() + 1
        logits = logits + skew * rank.pow(-1.1) * 4
    idx = torch.topk(logits, K, dim=-1).indices
    if sentinel_every:
        idx[::sentinel_every, -1] = E + 1
    return idx


@pytest.mark.parametrize("T,E,K,skew,sent", [
    (2048, 16, 4, 0.0, 0),
    (65536, 128, 8, 0.0, 0),      # L shape
    (32768, 128, 8, 2.0, 0),      # M shape, skewed
    (16384, 1792, 8, 0.0, 0),     # retrofit bank
    (1001, 64, 3, 0.0, 7),        # ragged S, sentinel ids
    (1, 8, 1, 0.0, 0),
])
def test_permute_parity(T, E, K, skew, sent):
    print(f"permute T={T} E={E} K={K} skew={skew} sentinels={sent}", flush=True)
    idx = _routing(T, E, K, T + E, skew, sent)
    plan = ops.permute(idx.to(DEV), E)
    torch.cuda.synchronize()
    ref = O.permute(idx, E)
    assert np.array_equal(plan.counts.cpu().numpy(), ref.counts)
    assert np.array_equal(plan.offsets.cpu().numpy(), ref.offsets)
    assert np.array_equal(plan.row_src.cpu().numpy(), ref.row_src)
    assert np.array_equal(plan.slot.cpu().numpy(), ref.slot)
    assert np.array_equal(plan.tile_starts.cpu().numpy(), ref.tile_starts)


def test_permute_empty_experts_and_determinism():
    T, E, K = 4096, 256, 2
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(0, 8, (T, K), generator=g) * 32  # only 8 experts used (may repeat)
    a = ops.permute(idx.to(DEV), E)
    b = ops.permute(idx.to(DEV), E)
    ref = O.permute(idx, E)
    assert np.array_equal(a.row_src.cpu().numpy(), ref.row_src)
    assert torch.equal(a.row_src, b.row_src) and torch.equal(a.slot, b.slot)
    assert int((a.counts > 0).sum()) <= 8


def test_permute_zero_tokens():
    idx = torch.empty(0, 4, dtype=torch.int64, device=DEV)
    plan = ops.permute(idx, 16)
    torch.cuda.synchronize()
    assert plan.offsets.cpu().tolist() == [0] * 17
    assert plan.counts.cpu().tolist() == [0] * 16
    assert plan.tile_starts.cpu().sum().item() == 0


@pytest.mark.parametrize("T,E,K", [(4096, 128, 8), (1001, 64, 3), (512, 1792, 8)])
def test_tile_plan_tables(T, E, K):
    """The {expert, first row, end row} table of every row tile, per tile height."""
    idx = _routing(T, E, K, 5 + E)
    plan = ops.permute(idx.to(DEV), E)
    torch.cuda.synchronize()
    ref = O.permute(idx, E)
    raw = plan.tile_plan.cpu().numpy()
    S = T * K
    # the row-tile height: least tiles x (BM + 256), the larger on ties
    cost = [int(ref.tile_starts[b, E]) * (bm + 256) for b, bm in enumerate(O.TILE_SIZES)]
    best = min(range(3), key=lambda b: (cost[b], -b))
    assert int(plan.row_tile.cpu()[0]) == best
    base = (3 * (E + 1) * 4 + 4 + 15) // 16 * 16
    for b, bm in enumerate(O.TILE_SIZES):
        ntile = int(ref.tile_starts[b, E])
        info = raw[base: base + 16 * ntile].view(np.int32).reshape(ntile, 4)[:, :3]
        exp = []
        for e in range(E):
            lo, hi = int(ref.offsets[e]), int(ref.offsets[e + 1])
            exp += [(e, r, hi) for r in range(lo, hi, bm)]
        assert info.tolist() == [list(x) for x in exp]
        base += 16 * ((S + bm - 1) // bm + E)
