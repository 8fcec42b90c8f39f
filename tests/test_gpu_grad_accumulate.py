"""Fused gradient accumulation of the expert weights on the GPU: the dW
GEMMs' accumulating forms (moe_amd_gemm_gate_up_backward_dw_accumulate,
moe_amd_gemm_down_backward_dw_gathered_accumulate) and a weight's main_grad
through the layers.

An expert bank shared by several layers (src/models/global_moe.py:138,
:147-151) gets its gradient from autograd: each layer's dense bf16 dW is
added to the bank's gradient, a bf16 add.  The accumulating forms must give
those bits: per element acc = bf16(acc + dW), dW the non-accumulating op's
output on the same device, the add done by torch.  Experts without routed
rows are neither read nor written: they are NaN-filled here and must keep
their bits.  Through the layers, a main_grad on the bank (the attribute name
Megatron-LM uses) must end equal to the gradient autograd accumulates for
the same two-layer use of the bank, with autograd's own .grad left None.
"""
from __future__ import annotations

import pytest
import torch

from moe_amd import experts_forward, ops
from moe_amd.layer import moe_layer
from test_gpu_experts import _check_sched

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16


def _routing(T, E, K, seed, skew=0.0, active=None):
    """top-K expert ids of random logits: Zipf-like skew, or only `active`
    randomly chosen experts reachable (the rest get no rows)."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=g)
    if skew:
        logits += skew * (torch.randperm(E, generator=g).float() + 1).pow(-1.1) * 8
    if active is not None:
        off = torch.full((E,), float("-inf"))
        off[torch.randperm(E, generator=g)[:active]] = 0.0
        logits += off
    return logits.topk(K, dim=-1).indices


def _bits(t):
    return t.view(torch.int16)


@pytest.mark.parametrize("T,H,E,K,I,skew,active", [
    (4096, 1024, 128, 8, 256, 3.0, None),   # Zipf-like skew, empty experts
    (1500, 512, 13, 4, 256, 2.0, None),     # E not a multiple of the 8 XCDs
    (700, 256, 5, 2, 256, 0.0, None),       # fewer experts than XCDs
    (2048, 512, 1792, 8, 256, 0.0, 355),    # a 1792-expert bank, 355 experts routed to
    (3, 128, 40, 2, 128, 0.0, None),        # fewer rows than experts
])
def test_dw_accumulate_matches_autograd_add(T, H, E, K, I, skew, active):
    print(f"dW accumulate T={T} H={H} E={E} K={K} I={I} skew={skew} active={active}", flush=True)
    idx = _routing(T, E, K, T + E, skew, active).to(DEV)
    plan = ops.permute(idx, E)
    S = T * K
    g = torch.Generator().manual_seed(E + 7)
    dgu = torch.randn(S, 2 * I, generator=g).to(BF).to(DEV)
    xd = torch.randn(T, H, generator=g).to(BF).to(DEV)
    dout = torch.randn(T, H, generator=g).to(BF).to(DEV)
    actw = torch.randn(S, I, generator=g).to(BF).to(DEV)
    ref1 = ops.gemm_gate_up_backward_dw(dgu, xd, plan, (E, 2 * I, H))
    ref2 = ops.gemm_down_backward_dw_gathered(dout, actw, plan, (E, H, I))
    empty = plan.counts == 0
    acc1 = (torch.randn(E, 2 * I, H, generator=g) * 4).to(BF).to(DEV)
    acc2 = (torch.randn(E, H, I, generator=g) * 4).to(BF).to(DEV)
    acc1[empty] = float("nan")
    acc2[empty] = float("nan")
    exp1, exp2 = acc1.clone(), acc2.clone()
    for call in range(2):  # the second call starts from the first's sums and reset queues
        exp1[~empty] += ref1[~empty]
        exp2[~empty] += ref2[~empty]
        ops.gemm_gate_up_backward_dw_accumulate(dgu, xd, plan, acc1)
        ops.gemm_down_backward_dw_gathered_accumulate(dout, actw, plan, acc2)
        torch.cuda.synchronize()
        assert torch.equal(_bits(acc1), _bits(exp1)), f"gate_up dW accumulation, call {call}"
        assert torch.equal(_bits(acc2), _bits(exp2)), f"down dW accumulation, call {call}"
    _check_sched(plan, S, E)


def test_dw_accumulate_rejects():
    """bf16, contiguous accumulators of the operands' weight shape only, and
    operands that match the plan and each other."""
    T, H, E, K, I = 64, 128, 8, 2, 64
    idx = _routing(T, E, K, 1).to(DEV)
    plan = ops.permute(idx, E)
    dgu = torch.zeros(T * K, 2 * I, dtype=BF, device=DEV)
    x = torch.zeros(T, H, dtype=BF, device=DEV)
    for acc in (torch.zeros(E, 2 * I, H, device=DEV),                     # fp32
                torch.zeros(E, 2 * I, H + 64, dtype=BF, device=DEV),        # shape
                torch.zeros(E, H, 2 * I, dtype=BF, device=DEV).transpose(1, 2)):  # layout
        with pytest.raises(ValueError, match="accumulator"):
            ops.gemm_gate_up_backward_dw_accumulate(dgu, x, plan, acc)
    acc = torch.zeros(E, 2 * I, H, dtype=BF, device=DEV)
    with pytest.raises(TypeError, match="dtypes"):                       # operand dtypes
        ops.gemm_gate_up_backward_dw_accumulate(dgu, x.float(), plan, acc)
    with pytest.raises(ValueError, match="plan"):                        # operand rows
        ops.gemm_gate_up_backward_dw_accumulate(dgu[:-1], x, plan, acc)


def _bank(E, H, I, seed):
    g = torch.Generator().manual_seed(seed)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(BF).to(DEV)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(BF).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(BF).to(DEV)
    bias = ((torch.rand(E, generator=g) * 2 - 1) * 0.5).to(DEV)
    xs = [torch.randn(T, H, generator=g).to(BF).to(DEV) for T in (700, 333)]
    douts = [torch.randn(T, H, generator=g).to(BF).to(DEV) for T in (700, 333)]
    return w1, w2, wr, bias, xs, douts


@pytest.mark.parametrize("path", ["experts", "softmax_layer", "sigmoid_layer"])
def test_main_grad_matches_autograd_accumulation(path):
    """Two layers share one bank (E=256, K=2: many experts without rows in
    each call).  With main_grad set (zeros), the backward leaves .grad None
    and main_grad equal to the .grad autograd accumulates without it; the
    input, router and routing-weight gradients are unchanged."""
    print(f"main_grad {path}", flush=True)
    E, H, I, K = 256, 512, 256, 2
    w1_0, w2_0, wr0, bias, xs, douts = _bank(E, H, I, 17)
    results = []
    for fused in (False, True):
        w1 = w1_0.clone().requires_grad_(True)
        w2 = w2_0.clone().requires_grad_(True)
        wr = wr0.clone().requires_grad_(True)
        if fused:
            w1.main_grad = torch.zeros_like(w1)
            w2.main_grad = torch.zeros_like(w2)
        leaves = []
        total = 0
        for x0, dout in zip(xs, douts):
            x = x0.clone().requires_grad_(True)
            leaves.append(x)
            if path == "experts":
                logits = x.float() @ wr.float().T
                wt, idx = torch.softmax(logits, -1).topk(K, dim=-1)
                wt = wt / wt.sum(-1, keepdim=True)
                out = experts_forward(x, idx, wt, w1, w2)
            elif path == "softmax_layer":
                out = moe_layer(x, wr, w1, w2, K, gating="hip")[0]
            else:
                out = moe_layer(x, wr, w1, w2, K, router="sigmoid", expert_bias=bias,
                                gating="hip")[0]
            total = total + (out.float() * dout.float()).sum()
        total.backward()
        torch.cuda.synchronize()
        if fused:
            assert w1.grad is None and w2.grad is None
            g1, g2 = w1.main_grad, w2.main_grad
        else:
            g1, g2 = w1.grad, w2.grad
        results.append((g1, g2, wr.grad) + tuple(t.grad for t in leaves))
    for a, b in zip(*results):
        assert torch.equal(a, b)


def test_main_grad_rejects_unusable_buffer():
    """A main_grad that the fused accumulation cannot use is an error, not
    silently ignored."""
    E, H, I, K = 16, 128, 64, 2
    w1_0, w2_0, wr0, _, xs, _ = _bank(E, H, I, 3)
    w1 = w1_0.clone().requires_grad_(True)
    w1.main_grad = torch.zeros(w1.shape, device=DEV)  # fp32
    with pytest.raises(ValueError, match="main_grad"):
        moe_layer(xs[0], wr0, w1, w2_0, K, gating="hip")
