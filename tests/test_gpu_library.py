"""The moe_amd:: custom ops on the GPU: torch.library.opcheck (schema, fake
implementation against the real op, autograd registration, AOT dispatch),
and the expert layer and the one-node softmax layer under
torch.compile(fullgraph=True) -- a graph break would fail the compile --
giving bit-identical outputs and gradients to eager execution."""
from __future__ import annotations

import pytest
import torch

import moe_amd  # noqa: F401
from moe_amd.experts import experts_forward
from moe_amd.layer import moe_layer
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
# test_aot_dispatch_dynamic is left out: the tile plan's size is a host
# function of S and E that becomes an unbacked size under symbolic shapes,
# which the dynamic-shape check cannot compare against the real op.
UTILS = ("test_schema", "test_autograd_registration", "test_faketensor",
         "test_aot_dispatch_static")


def _inputs(T=512, H=256, E=16, K=4, I=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    _, w, idx = O.softmax_router(x.float() @ wr.float().T, K)
    dout = torch.randn(T, H, generator=g).to(torch.bfloat16)
    return [t.to(DEV) for t in (x, wr, w1, w2, w, idx, dout)]


def test_opcheck_experts():
    print("opcheck experts_fwd", flush=True)
    x, _, w1, w2, w, idx, _ = _inputs()
    args = (x.requires_grad_(True), idx, w.requires_grad_(True), w1.requires_grad_(True),
            w2.requires_grad_(True), True)
    torch.library.opcheck(torch.ops.moe_amd.experts_fwd.default, args, test_utils=UTILS)


def test_opcheck_routers():
    print("opcheck routers", flush=True)
    x, wr, *_ = _inputs()
    logits = torch.ops.moe_amd.router_linear(x, wr, torch.bfloat16).detach()
    torch.library.opcheck(torch.ops.moe_amd.router_linear.default,
                          (x.requires_grad_(True), wr.requires_grad_(True), torch.float32),
                          test_utils=UTILS)
    for fp32 in (True, False):
        torch.library.opcheck(torch.ops.moe_amd.torch_gating_linear.default,
                              (x.detach().requires_grad_(True), wr.detach().requires_grad_(True),
                               fp32), test_utils=UTILS)
    torch.library.opcheck(torch.ops.moe_amd.softmax_topk.default,
                          (logits.requires_grad_(True), 4, True, None), test_utils=UTILS)
    f32 = logits.detach().float().requires_grad_(True)
    bias = torch.rand(f32.shape[1], device=DEV) - 0.5
    torch.library.opcheck(torch.ops.moe_amd.sigmoid_topk.default,
                          (f32, bias, 4, True, 0.0, 0, 0, torch.bfloat16, True), test_utils=UTILS)


@pytest.mark.parametrize("gating", ["torch", "hip"])
def test_opcheck_layer(gating):
    print(f"opcheck moe_layer_fwd gating={gating}", flush=True)
    x, wr, w1, w2, *_ = _inputs()
    args = tuple(t.requires_grad_(True) for t in (x, wr, w1, w2)) + (4, True, None, True, gating)
    torch.library.opcheck(torch.ops.moe_amd.moe_layer_fwd.default, args, test_utils=UTILS)


def _run(fn, x, wr, w1, w2, w, idx, dout):
    leaves = [t.detach().clone().requires_grad_(True) for t in (x, wr, w1, w2, w)]
    outs = fn(*leaves, idx)
    outs[0].backward(dout)
    return [o.detach() for o in outs] + [t.grad for t in leaves if t.grad is not None]


@pytest.mark.parametrize("layer", [False, True])
def test_compile_fullgraph_matches_eager(layer):
    """torch.compile(fullgraph=True, backend="aot_eager"): one graph (no
    break) that runs the same HIP kernels; results bit-identical to eager."""
    print(f"compile fullgraph layer={layer}", flush=True)
    torch._dynamo.reset()
    x, wr, w1, w2, w, idx, dout = _inputs(seed=3)

    def f(x, wr, w1, w2, w, idx):
        if layer:
            out, probs, wt, ix = moe_layer(x, wr, w1, w2, 4)
            return out, probs
        return (experts_forward(x, idx, w, w1, w2),)

    eager = _run(f, x, wr, w1, w2, w, idx, dout)
    comp = _run(torch.compile(f, fullgraph=True, backend="aot_eager"), x, wr, w1, w2, w, idx,
                dout)
    torch.cuda.synchronize()
    assert len(eager) == len(comp)
    for a, b in zip(eager, comp):
        assert torch.equal(a, b)


def test_layer_backward_overlap_matches_in_order():
    """The softmax layer's backward with the gather backward on a second
    stream (beside the weight-gradient GEMMs) gives the same bits as with
    every kernel in order on one stream (the per-launch timing mode), on
    three steps in a row."""
    from moe_amd import ops
    print("backward overlap vs in order", flush=True)
    x, wr, w1, w2, _, _, dout = _inputs(T=4096, H=512, E=32, K=4, I=256, seed=7)
    grads = []
    for timed in (True, False, False, False):
        leaves = [t.detach().clone().requires_grad_(True) for t in (x, wr, w1, w2)]
        if timed:
            ops.record_kernel_times([])
        try:
            out, *_ = moe_layer(*leaves, 4)
            out.backward(dout)
        finally:
            ops.record_kernel_times(None)
        torch.cuda.synchronize()
        grads.append([t.grad.clone() for t in leaves])
    for g in grads[1:]:
        for a, b in zip(grads[0], g):
            assert torch.equal(a, b)


def test_experts_backward_overlap_matches_in_order():
    """The same for the expert-layer op (the ExpertsInterface path)."""
    from moe_amd import ops
    print("experts backward overlap vs in order", flush=True)
    x, _, w1, w2, w, idx, dout = _inputs(T=4096, H=512, E=32, K=4, I=256, seed=8)
    grads = []
    for timed in (True, False, False):
        leaves = [t.detach().clone().requires_grad_(True) for t in (x, w, w1, w2)]
        if timed:
            ops.record_kernel_times([])
        try:
            out = experts_forward(leaves[0], idx, leaves[1], leaves[2], leaves[3])
            out.backward(dout)
        finally:
            ops.record_kernel_times(None)
        torch.cuda.synchronize()
        grads.append([t.grad.clone() for t in leaves])
    for g in grads[1:]:
        for a, b in zip(grads[0], g):
            assert torch.equal(a, b)
