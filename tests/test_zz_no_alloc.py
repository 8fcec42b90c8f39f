"""moe_amd_permute_noalloc (the allocation-free permutation, scratch in a
static device array) against moe_amd_permute (caller workspace), both called
through the C ABI: every output bit-identical, on two calls in a row with the
second on a smaller input (the array keeps the first call's contents), and
the size limit refused with a clear error."""
from __future__ import annotations

import pytest
import torch

from moe_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _outputs(S, E):
    lib = _lib.load()
    i32 = dict(device=DEV, dtype=torch.int32)
    plan_bytes = int(lib.moe_amd_tile_plan_size(S, E))
    return (torch.full((E,), -7, **i32), torch.full((E + 1,), -7, **i32),
            torch.full((S,), -7, **i32), torch.full((S,), -7, **i32),
            torch.zeros(plan_bytes, device=DEV, dtype=torch.uint8))


def _run(idx, E, noalloc):
    lib = _lib.load()
    S = idx.numel()
    counts, offsets, row_src, slot, plan = _outputs(S, E)
    st = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.moe_amd_permute_noalloc(idx.data_ptr(), S, E, counts.data_ptr(),
                                         offsets.data_ptr(), row_src.data_ptr(), slot.data_ptr(),
                                         plan.data_ptr(), plan.numel(), st)
    else:
        ws = torch.empty(max(int(lib.moe_amd_permute_workspace_size(S, E)), 256), device=DEV,
                         dtype=torch.uint8)
        rc = lib.moe_amd_permute(idx.data_ptr(), S, E, ws.data_ptr(), ws.numel(),
                                 counts.data_ptr(), offsets.data_ptr(), row_src.data_ptr(),
                                 slot.data_ptr(), plan.data_ptr(), plan.numel(), st)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return counts, offsets, row_src, slot, plan


def test_permute_noalloc_matches_permute():
    g = torch.Generator().manual_seed(0)
    # first call large (the L layer's routing shape), second smaller, skewed,
    # with EP sentinels: the array holds the first call's data when the
    # second starts
    cases = [(65536, 8, 128, False), (3001, 4, 1792, True)]
    for T, K, E, sentinels in cases:
        print(f"permute_noalloc T={T} K={K} E={E} sentinels={sentinels}", flush=True)
        if sentinels:
            idx = (torch.rand(T, K, generator=g).pow(3) * E).long()
            idx[::5, -1] = E
        else:
            idx = torch.randint(0, E, (T, K), generator=g)
        idx = idx.to(DEV)
        ref = _run(idx, E, noalloc=False)
        got = _run(idx, E, noalloc=True)
        for name, a, b in zip(("counts", "offsets", "row_src", "slot", "tile_plan"), got, ref):
            assert torch.equal(a, b), name


def test_permute_noalloc_refuses_oversize():
    lib = _lib.load()
    S, E = 1 << 30, 1024  # needs far more than the static array
    assert lib.moe_amd_permute_workspace_size(S, E) > 8 << 20
    rc = lib.moe_amd_permute_noalloc(None, S, E, None, None, None, None, None, 0, None)
    assert rc == -6 and "static array" in _lib.last_error()
