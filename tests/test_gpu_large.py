"""Routed-row buffers larger than 4 GiB: the expert layer at the L shape
(H=2048, E=128, K=8, I=768) with T = 147456 tokens, S = T*K = 1179648
routed rows, so [S, H] bf16 buffers hold 4.8 GB.  Every per-token result
(output, d_x, d_topk_weights) must be bit-identical to the same layer run
on the two halves of the batch (each below 4 GiB), since a row's
arithmetic does not depend on the other rows; the weight gradients, which
sum over all rows, must match the sum of the halves' to bf16 rounding."""
from __future__ import annotations

import pytest
import torch

import moe_amd  # noqa: F401
from moe_amd.experts import experts_forward

pytestmark = pytest.mark.gpu
DEV = "cuda"
T, H, E, K, I = 147456, 2048, 128, 8, 768


def _run(x, idx, w, w1, w2, dout):
    leaves = [t.detach().clone().requires_grad_(True) for t in (x, w, w1, w2)]
    out = experts_forward(leaves[0], idx, leaves[1], leaves[2], leaves[3])
    out.backward(dout)
    torch.cuda.synchronize()
    return out.detach(), [t.grad for t in leaves]


def test_routed_rows_beyond_4gib_match_halves():
    S = T * K
    assert S * max(H, 2 * I) * 2 >= 1 << 32  # past the former per-call limit
    print(f"large S: T={T} S={S} H={H} E={E} K={K} I={I}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(11)
    x = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(E, 2 * I, H, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    logits = torch.randn(T, E, device=DEV, generator=g)
    top, idx = logits.topk(K, dim=1)  # distinct experts per token
    w = torch.softmax(top, dim=1).to(torch.bfloat16)
    dout = torch.randn(T, H, device=DEV, generator=g).to(torch.bfloat16)

    out, (dx, dw, dw1, dw2) = _run(x, idx, w, w1, w2, dout)
    h = T // 2
    parts = [_run(x[a:b], idx[a:b], w[a:b], w1, w2, dout[a:b]) for a, b in ((0, h), (h, T))]
    print("large S: compared with the halves", flush=True)
    assert torch.equal(out, torch.cat([p[0] for p in parts]))
    assert torch.equal(dx, torch.cat([p[1][0] for p in parts]))
    assert torch.equal(dw, torch.cat([p[1][1] for p in parts]))
    for full, a, b in ((dw1, parts[0][1][2], parts[1][1][2]), (dw2, parts[0][1][3], parts[1][1][3])):
        ref = a.float() + b.float()
        err = (full.float() - ref).abs().max() / ref.abs().max()
        assert err < 1e-2, float(err)


@pytest.mark.parametrize("gemm", ["gate_up_dw", "down_dw_gathered"])
def test_dw_expert_rows_beyond_4gib(gemm):
    """Every token lists expert 0 in all K slots (accepted: the reference's
    grouped_mm path does not require distinct ids), so expert 0 owns all
    S = T*K routed rows and its k-major row operand -- d_gate_up [S, 2I] or
    act_w [S, I] -- spans more than 4 GiB in one dW tile's k walk.  The
    weight gradient must equal torch's fp32 product of the same bf16
    operands (rows gathered through row_src) to the bf16 rounding of the
    result; expert 1, with no rows, gets exact zeros."""
    from moe_amd import ops
    Hs, Is, Es, Ks = 256, 768, 2, 8
    ld = 2 * Is if gemm == "gate_up_dw" else Is
    Ts = ((1 << 32) // (ld * 2) + 4096) // Ks + 1
    S = Ts * Ks
    assert S * ld * 2 > 1 << 32
    print(f"dW rows past 4 GiB: {gemm} T={Ts} S={S} ld={ld}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    idx = torch.zeros(Ts, Ks, dtype=torch.int64, device=DEV)
    plan = ops.permute(idx, Es)
    a = torch.randn(S, ld, device=DEV, generator=g).to(torch.bfloat16)
    rows = torch.randn(Ts, Hs, device=DEV, generator=g).to(torch.bfloat16)
    tok = plan.row_src.long() // Ks
    if gemm == "gate_up_dw":
        dw = ops.gemm_gate_up_backward_dw(a, rows, plan, (Es, 2 * Is, Hs))
        ref = a.float().t() @ rows[tok].float()            # [2I, H]
    else:
        dw = ops.gemm_down_backward_dw_gathered(rows, a, plan, (Es, Hs, Is))
        ref = rows[tok].float().t() @ a.float()            # [H, I]
    torch.cuda.synchronize()
    err = ((dw[0].float() - ref).abs().max() / ref.abs().max()).item()
    print(f"  max rel err {err:.2e}", flush=True)
    assert err < 1e-2
    assert not dw[1].any()
