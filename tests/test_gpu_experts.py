"""GPU parity of the expert layer (grouped GEMMs, SwiGLU, combine and the
full backward) against the CPU oracle on the same seeded inputs.

Tolerance (bf16): max |gpu - oracle| / max |oracle| <= 2e-2 per tensor; in
practice the oracle reproduces every bf16 rounding point, so the two differ
only by fp32 accumulation order.  Full-size (L shape) checks use
size-independent properties: per-token outputs and input gradients of a
random token sample, and the weight gradients of sampled experts, each
recomputed by the oracle from exactly the tokens that determine them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from moe_amd import experts_forward, ops
from moe_amd.configs import CONFIGS, make_inputs
from moe_amd.layer import moe_layer
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2e-2


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def _inputs(T, H, E, K, I, seed=0, skew=0.0, sentinel_every=0, w_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    wr = (torch.randn(E, H, generator=g) * 0.02)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    logits = x.float() @ wr.T
    if skew:
        rank = torch.randperm(E, generator=g).float() + 1
        logits = logits + skew * rank.pow(-1.1) * 8
    _, w, idx = O.softmax_router(logits, K)
    if sentinel_every:
        idx[::sentinel_every, -1] = E
    dout = torch.randn(T, H, generator=g).to(torch.bfloat16)
    return x, idx, w.to(w_dtype), w1, w2, dout


CASES = [
    # T, H, E, K, I, skew, sentinels, weights dtype
    (1024, 1024, 16, 4, 768, 0.0, 0, torch.float32),    # XS shape, small T
    (2048, 512, 64, 8, 256, 3.0, 0, torch.float32),     # heavy skew, empty experts
    (777, 256, 32, 2, 128, 0.0, 5, torch.float32),      # ragged T, EP sentinels
    (600, 512, 256, 8, 192, 0.0, 0, torch.bfloat16),    # tiny groups, bf16 weights
    (901, 320, 24, 3, 320, 1.0, 7, torch.float32),      # H, I, 2I not multiples of 256
    (513, 64, 1, 1, 64, 0.0, 0, torch.float32),         # one expert, top-1, smallest H and I
    (300, 128, 8, 1, 64, 0.0, 0, torch.bfloat16),       # top-1 routing
    (200, 256, 4, 4, 128, 0.0, 0, torch.float32),       # K = E: every token to every expert
]


@pytest.mark.parametrize("T,H,E,K,I,skew,sent,wdt", CASES)
def test_forward_kernels_parity(T, H, E, K, I, skew, sent, wdt):
    print(f"forward kernels T={T} H={H} E={E} K={K} I={I} skew={skew} sent={sent} {wdt}",
          flush=True)
    x, idx, w, w1, w2, _ = _inputs(T, H, E, K, I, T + E, skew, sent, wdt)
    out_ref, cache = O.experts_forward(x, idx, w, w1, w2)
    plan = ops.permute(idx.to(DEV), E)
    gu, act = ops.gemm_gate_up_swiglu(x.to(DEV), plan, w1.to(DEV), save_gate_up=True)
    y = ops.gemm_down(act, plan, w2.to(DEV))
    out = ops.combine(y, plan, w.to(DEV))
    torch.cuda.synchronize()
    nv = int(cache["plan"].offsets[E])
    assert _rel(gu[:nv], cache["gate_up"][:nv]) < TOL
    assert _rel(act[:nv], cache["act"][:nv]) < TOL
    assert _rel(y[:nv], cache["y"][:nv]) < TOL
    assert _rel(out, out_ref) < TOL
    # act without the gate_up side output is identical
    _, act2 = ops.gemm_gate_up_swiglu(x.to(DEV), plan, w1.to(DEV), save_gate_up=False)
    assert torch.equal(act2[:nv], act[:nv])  # sentinel rows are never written


@pytest.mark.parametrize("T,H,E,K,I,skew,sent,wdt", CASES)
def test_backward_parity(T, H, E, K, I, skew, sent, wdt):
    print(f"backward T={T} H={H} E={E} K={K} I={I} skew={skew} sent={sent} {wdt}", flush=True)
    x, idx, w, w1, w2, dout = _inputs(T, H, E, K, I, T + E + 1, skew, sent, wdt)
    out_ref, cache = O.experts_forward(x, idx, w, w1, w2)
    dx_ref, dw_ref, dw1_ref, dw2_ref, inter = O.experts_backward(cache, x, w, w1, w2, dout)
    xs, ws, w1s, w2s = (t.to(DEV).requires_grad_(True) for t in (x, w, w1, w2))
    out = experts_forward(xs, idx.to(DEV), ws, w1s, w2s)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    assert _rel(out, out_ref) < TOL
    assert xs.grad.dtype == torch.bfloat16 and ws.grad.dtype == wdt
    assert _rel(xs.grad, dx_ref) < TOL
    assert _rel(ws.grad, dw_ref) < TOL
    assert _rel(w1s.grad, dw1_ref) < TOL
    assert _rel(w2s.grad, dw2_ref) < TOL
    used = set(idx[idx < E].reshape(-1).tolist())
    for e in range(E):
        if e not in used:
            assert w1s.grad[e].abs().max().item() == 0 and w2s.grad[e].abs().max().item() == 0


@pytest.mark.parametrize("T,H,E,K,I,skew,sent,wdt", CASES)
def test_down_backward_fused_parity(T, H, E, K, I, skew, sent, wdt):
    """The combine backward fused into GEMM-2's backward (d_out rows gathered
    by token, no d_y): d_gate_up, the routing-weight gradient and d_down_proj
    against the oracle (which rounds d_y = w * d_out as the reference does;
    the fused path rounds g = d_out . down_proj instead, hence the tolerance),
    and the side output act_w bit-exact to w * act."""
    print(f"fused down backward T={T} H={H} E={E} K={K} I={I} skew={skew} sent={sent} {wdt}",
          flush=True)
    x, idx, w, w1, w2, dout = _inputs(T, H, E, K, I, T + E + 2, skew, sent, wdt)
    _, cache = O.experts_forward(x, idx, w, w1, w2)
    _, dw_ref, _, dw2_ref, inter = O.experts_backward(cache, x, w, w1, w2, dout)
    plan = ops.permute(idx.to(DEV), E)
    gu, act = ops.gemm_gate_up_swiglu(x.to(DEV), plan, w1.to(DEV))
    wd, dd = w.to(DEV), dout.to(DEV)
    d_gu, act_w, dw = ops.gemm_down_backward_fused(dd, plan, w2.to(DEV), gu, wd)
    d_w2 = ops.gemm_down_backward_dw_gathered(dd, act_w, plan, w2.shape)
    d_w2s = ops.gemm_down_backward_dw_gathered(dd, act_w, plan, w2.shape, scheduled=False)
    torch.cuda.synchronize()
    nv = int(cache["plan"].offsets[E])
    wrow = wd.reshape(-1)[plan.row_src[:nv].long()].float()
    assert torch.equal(act_w[:nv], (act[:nv].float() * wrow[:, None]).to(torch.bfloat16))
    assert dw.dtype == wdt
    assert _rel(dw, dw_ref) < TOL
    if sent:
        assert not dw.cpu()[idx >= E].any()        # sentinel entries: zero gradient
    assert _rel(d_gu[:nv], inter["d_gate_up"][:nv]) < TOL
    assert _rel(d_w2, dw2_ref) < TOL
    assert torch.equal(d_w2, d_w2s)               # claimed and static tile walks agree


def test_layer_deterministic_and_drop_in_shapes():
    """Two identical fwd+bwd calls give bitwise-identical results."""
    x, idx, w, w1, w2, dout = _inputs(1536, 512, 32, 4, 256, seed=9)
    res = []
    for _ in range(2):
        xs, ws, w1s, w2s = (t.to(DEV).requires_grad_(True) for t in (x, w, w1, w2))
        out = experts_forward(xs, idx.to(DEV), ws, w1s, w2s)
        out.backward(dout.to(DEV))
        res.append([out, xs.grad, ws.grad, w1s.grad, w2s.grad])
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_l_shape_sampled_parity():
    """L (Qwen3-30B-A3B) shape end to end on the full T=65536 batch: routing
    bit-exact for every token; outputs, dX and d(weights) on a 256-token
    sample; dW of the most- and least-loaded experts from all their tokens."""
    from moe_amd.router import softmax_topk
    cfg = CONFIGS["l"]
    print("L shape sampled parity", flush=True)
    inp = make_inputs(cfg, seed=0, device=DEV)
    logits = F.linear(inp.x, inp.w_router)
    _, w, idx = softmax_topk(logits, cfg.K, True, None)
    xe = inp.x.clone().requires_grad_(True)
    wl = w.detach().clone().requires_grad_(True)
    w1 = inp.gate_up_proj.clone().requires_grad_(True)
    w2 = inp.down_proj.clone().requires_grad_(True)
    out = experts_forward(xe, idx, wl, w1, w2)
    out.backward(inp.dout)
    torch.cuda.synchronize()
    _, w_ref, i_ref = O.softmax_router(logits.cpu(), cfg.K)
    assert torch.equal(idx.cpu(), i_ref), "L-shape routing differs"
    assert torch.allclose(w.cpu(), w_ref, rtol=1e-5, atol=1e-7)
    counts = torch.bincount(i_ref.reshape(-1), minlength=cfg.E)
    g = torch.Generator().manual_seed(1)
    sample = torch.randperm(cfg.T, generator=g)[:256]
    w1c, w2c = inp.gate_up_proj.cpu(), inp.down_proj.cpu()
    xs_cpu, ws_cpu = inp.x[sample].cpu(), w_ref[sample]
    o_ref, cache = O.experts_forward(xs_cpu, i_ref[sample], ws_cpu, w1c, w2c)
    dx_ref, dw_ref, _, _, _ = O.experts_backward(cache, xs_cpu, ws_cpu, w1c, w2c,
                                                 inp.dout[sample].cpu())
    assert _rel(out.detach()[sample], o_ref) < TOL
    assert _rel(xe.grad[sample], dx_ref) < TOL
    assert _rel(wl.grad[sample], dw_ref) < TOL
    for e in (int(counts.argmax()), int(counts.argmin())):
        toks = (i_ref == e).any(-1).nonzero().flatten()
        xt, wt = inp.x[toks].cpu(), w_ref[toks]
        _, c2 = O.experts_forward(xt, i_ref[toks], wt, w1c, w2c)
        _, _, dw1_ref, dw2_ref, _ = O.experts_backward(c2, xt, wt, w1c, w2c, inp.dout[toks].cpu())
        assert _rel(w1.grad[e], dw1_ref[e]) < TOL
        assert _rel(w2.grad[e], dw2_ref[e]) < TOL


def test_full_layer_router_gradient_flows():
    """moe_layer (gate linear + router kernel + experts) backpropagates into
    the router weight and the hidden states, matching the oracle's router
    backward for the dlogits it receives."""
    cfg = CONFIGS["xs_global"].scaled(2048)
    inp = make_inputs(cfg, seed=0, device=DEV)
    x = inp.x.clone().requires_grad_(True)
    wr = inp.w_router.clone().requires_grad_(True)
    out, probs, w, idx = moe_layer(x, wr, inp.gate_up_proj, inp.down_proj, cfg.K)
    out.backward(inp.dout)
    torch.cuda.synchronize()
    assert torch.isfinite(wr.grad).all() and wr.grad.abs().max() > 0
    assert torch.isfinite(x.grad).all()


def test_hip_gating_linear_matches_torch_gating():
    """moe_layer with the MFMA gating linear against the same layer with torch's
    F.linear (the reference's gating): the logits differ only in fp32 summation
    order before the bf16 rounding, so the top-k sets agree except on
    near-tied experts (bounded here at 0.5% of tokens at the L router shape),
    the outputs agree on the tokens routed identically, and the router-weight
    gradients agree within bf16 tolerance."""
    cfg = CONFIGS["l"].scaled(8192)
    inp = make_inputs(cfg, seed=0, device=DEV)
    res = {}
    for gating in ("hip", "torch"):
        x = inp.x.clone().requires_grad_(True)
        wr = inp.w_router.clone().requires_grad_(True)
        out, probs, w, idx = moe_layer(x, wr, inp.gate_up_proj, inp.down_proj, cfg.K,
                                       gating=gating)
        out.backward(inp.dout)
        res[gating] = (out.detach(), probs, idx, wr.grad, x.grad)
    torch.cuda.synchronize()
    o_h, p_h, i_h, g_h, dx_h = res["hip"]
    o_t, p_t, i_t, g_t, dx_t = res["torch"]
    same = (i_h.sort(dim=1).values == i_t.sort(dim=1).values).all(dim=1)
    frac = 1.0 - same.float().mean().item()
    print(f"tokens with a different top-{cfg.K} set: {frac * 100:.3f}%", flush=True)
    assert frac < 5e-3
    assert _rel(p_h, p_t) < 2e-2
    assert _rel(o_h[same], o_t[same]) < 2e-2
    assert _rel(g_h, g_t) < 5e-2
    assert _rel(dx_h[same], dx_t[same]) < 5e-2


def test_fused_softmax_layer_matches_composed_nodes():
    """The one-node softmax layer (op moe_amd::moe_layer_fwd, chosen by
    moe_layer for bf16 inputs) against the same arithmetic as three autograd
    nodes (router_linear -> softmax_topk -> experts_fwd): the forward, the
    expert-weight and router-weight gradients are bit-identical; d_x differs
    only through the gating linear's dX summation order (MFMA kernel vs
    torch), i.e. within one bf16 rounding of the router term."""
    from moe_amd.router import router_linear, softmax_topk
    cfg = CONFIGS["l"].scaled(4096)
    inp = make_inputs(cfg, seed=1, device=DEV)
    outs = []
    for fused in (True, False):
        x = inp.x.clone().requires_grad_(True)
        wr = inp.w_router.clone().requires_grad_(True)
        w1 = inp.gate_up_proj.clone().requires_grad_(True)
        w2 = inp.down_proj.clone().requires_grad_(True)
        if fused:
            out, probs, w, idx = moe_layer(x, wr, w1, w2, cfg.K, gating="hip")
        else:
            logits = router_linear(x, wr, torch.bfloat16)
            probs, w, idx = softmax_topk(logits, cfg.K, True, None)
            out = experts_forward(x, idx, w, w1, w2)
        out.backward(inp.dout)
        outs.append((out.detach(), probs, idx, x.grad, wr.grad, w1.grad, w2.grad))
    torch.cuda.synchronize()
    a, b = outs
    for i in (0, 1, 2, 4, 5, 6):
        assert torch.equal(a[i], b[i]), i
    assert _rel(a[3], b[3]) < 1e-2


def test_router_linear_backward_dx_and_gather_add():
    """The gating linear's dX kernel against fp32 torch (within one bf16
    rounding), and the gather backward with an addend against
    bf16(bf16(sum_k dxs[slot]) + addend), bit-exact."""
    g = torch.Generator().manual_seed(7)
    T, H, E, K = 4096, 2048, 128, 8
    dl = torch.randn(T, E, generator=g).to(torch.bfloat16).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    dx = ops.router_linear_backward_dx(dl, wr)
    ref = dl.float() @ wr.float()
    err = (dx.double() - ref.double()).abs()
    assert bool((err <= ref.double().abs() * 2.0 ** -8 + 1e-5 * ref.abs().max().item()).all())
    idx = torch.randint(0, E, (T, K), generator=g).to(DEV)
    plan = ops.permute(idx, E)
    dxs = torch.randn(T * K, H, generator=g).to(torch.bfloat16).to(DEV)
    add = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    got = ops.gather_backward(dxs, plan, addend=add)
    plain = ops.gather_backward(dxs, plan)
    want = (plain.float() + add.float()).to(torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("T,H,E", [(65536, 2048, 128), (1001, 512, 16), (37, 256, 8), (0, 256, 8),
                                   (4096, 768, 256), (3000, 512, 1792), (700, 256, 264)])
def test_router_linear_backward_dw(T, H, E):
    """The gating linear's weight gradient (split over token chunks, fp32
    partials) against fp32 torch on the same bf16 inputs: within one bf16
    rounding of each element plus 1e-5 of the largest; run twice, bit-equal
    (the chunk reduction order is fixed)."""
    print(f"router dW T={T} H={H} E={E}", flush=True)
    g = torch.Generator().manual_seed(T + H + E)
    dl = torch.randn(T, E, generator=g).to(torch.bfloat16).to(DEV)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    dw = ops.router_linear_backward_dw(dl, x)
    dw2 = ops.router_linear_backward_dw(dl, x)
    ref = dl.float().t().contiguous() @ x.float()
    torch.cuda.synchronize()
    assert dw.shape == (E, H) and dw.dtype == torch.bfloat16
    assert torch.equal(dw, dw2)
    err = (dw.double() - ref.double()).abs()
    tol = ref.double().abs() * 2.0 ** -8 + 1e-5 * max(ref.abs().max().item(), 1.0)
    assert bool((err <= tol).all()), float((err - tol).max())


@pytest.mark.parametrize("T,H,E,need", [(16384, 2048, 1792, "both"), (4096, 1024, 128, "both"),
                                        (1001, 512, 32, "x"), (777, 256, 96, "w"),
                                        (0, 256, 64, "both")])
def test_router_linear_backward_f32(T, H, E, need):
    """Gradients of the fp32 gating linear F.linear(h.float(), W.float()) from
    the two-term bf16 split of d_logits on the MFMA kernels, against fp64
    products of the same inputs: |got - exact| <= 2^-8 |exact| (the one bf16
    rounding) + 2^-14 sum|g||w| (the split's 2^-18 residual and fp32 sums);
    and equal to torch's fp32 GEMM + bf16 cast on >= 98% of the elements (the
    rest sit at a bf16 rounding boundary).  A gradient not asked for is not
    computed."""
    print(f"router f32 backward T={T} H={H} E={E} need={need}", flush=True)
    g = torch.Generator().manual_seed(T + H + E + 3)
    # sigmoid-derivative-sized gradients with a wide exponent range
    dl = (torch.randn(T, E, generator=g) * torch.rand(T, E, generator=g).pow(4) * 0.25).to(DEV)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    dx, dw = ops.router_linear_backward_f32(dl, x, wr, need != "w", need != "x")
    dx2, dw2 = ops.router_linear_backward_f32(dl, x, wr, need != "w", need != "x")
    torch.cuda.synchronize()
    assert torch.equal(dx, dx2) and torch.equal(dw, dw2)
    checks = []
    if need != "w":
        assert dx.shape == (T, H) and dx.dtype == torch.bfloat16
        exact = dl.double() @ wr.double()
        scale = dl.double().abs() @ wr.double().abs()
        fp32 = (dl @ wr.float()).to(torch.bfloat16)
        checks.append((dx, exact, scale, fp32))
    else:
        assert dx.numel() == 0
    if need != "x":
        assert dw.shape == (E, H) and dw.dtype == torch.bfloat16
        exact = dl.double().t() @ x.double()
        scale = dl.double().abs().t() @ x.double().abs()
        fp32 = (dl.t().contiguous() @ x.float()).to(torch.bfloat16)
        checks.append((dw, exact, scale, fp32))
    else:
        assert dw.numel() == 0
    for got, exact, scale, fp32 in checks:
        err = (got.double() - exact).abs()
        tol = exact.abs() * 2.0 ** -8 + scale * 2.0 ** -14
        assert bool((err <= tol).all()), float((err - tol).max())
        if got.numel():
            assert (got == fp32).double().mean().item() >= 0.98
    if T == 0 and need != "x":
        assert not dw.any()


def _sched_tables(plan, S, E):
    """(queue[2][16], xstart[9], xnz[8], xorder[E]) read back from the tile
    plan."""
    raw = plan.tile_plan.cpu().numpy()
    off = (3 * (E + 1) * 4 + 15) // 16 * 16
    for bm in (64, 128, 256):
        off += 16 * ((S + bm - 1) // bm + E)
    v = raw[off: off + 4 * (64 + E)].view(np.int32)
    return v[:32].reshape(2, 16), v[32:41], v[48:56], v[64:64 + E]


def _check_sched(plan, S, E):
    """The dW schedule tables are well-formed: reset queue counters, every
    expert once, balanced XCD ranges, each XCD's experts with rows first
    (xnz of them) and the serpentine bound on the XCDs' rows.  Returns the
    per-XCD rows."""
    queue, xstart, xnz, xorder = _sched_tables(plan, S, E)
    assert not queue.any()                       # reset after each launch
    assert sorted(xorder.tolist()) == list(range(E))
    n = np.diff(xstart)
    assert xstart[0] == 0 and xstart[8] == E and n.max() - n.min() <= 1
    counts = plan.counts.cpu().numpy()
    for i in range(8):
        lst = counts[xorder[xstart[i]:xstart[i + 1]]]
        assert (lst[:xnz[i]] > 0).all() and not lst[xnz[i]:].any()
    load = [counts[xorder[xstart[i]:xstart[i + 1]]].sum() for i in range(8)]
    assert max(load) <= sum(load) / 8 + counts.max() + 1   # serpentine dealing bound
    return load


@pytest.mark.parametrize("T,H,E,K,I,skew", [
    (4096, 1024, 128, 8, 256, 3.0),   # Zipf-like skew, empty experts
    (1500, 512, 13, 4, 256, 2.0),     # E not a multiple of the 8 XCDs
    (700, 256, 5, 2, 256, 0.0),       # fewer experts than XCDs
])
def test_dw_schedule_matches_static_walk(T, H, E, K, I, skew):
    """The dW GEMMs' claimed-tile schedule covers every tile exactly once,
    the zero tiles of the experts without rows included: bit-identical to the
    static walk, on two launches in a row (the last workgroup resets the
    queue counters) into NaN-filled outputs, with balanced, well-formed
    tables."""
    print(f"dW schedule T={T} H={H} E={E} K={K} I={I} skew={skew}", flush=True)
    x, idx, w, w1, w2, _ = _inputs(T, H, E, K, I, T + E + 3, skew)
    S = T * K
    plan = ops.permute(idx.to(DEV), E)
    g = torch.Generator().manual_seed(E)
    dy = torch.randn(S, H, generator=g).to(torch.bfloat16).to(DEV)
    act = torch.randn(S, I, generator=g).to(torch.bfloat16).to(DEV)
    dgu = torch.randn(S, 2 * I, generator=g).to(torch.bfloat16).to(DEV)
    xd = x.to(DEV)
    dout = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    ref2 = ops.gemm_down_backward_dw(dy, act, plan, (E, H, I), scheduled=False)
    ref1 = ops.gemm_gate_up_backward_dw(dgu, xd, plan, (E, 2 * I, H), scheduled=False)
    ref3 = ops.gemm_down_backward_dw_gathered(dout, act, plan, (E, H, I), scheduled=False)
    nan = float("nan")
    for _ in range(2):
        d2 = ops.gemm_down_backward_dw(dy, act, plan, (E, H, I), out=torch.full_like(ref2, nan))
        d1 = ops.gemm_gate_up_backward_dw(dgu, xd, plan, (E, 2 * I, H),
                                          out=torch.full_like(ref1, nan))
        d3 = ops.gemm_down_backward_dw_gathered(dout, act, plan, (E, H, I),
                                                out=torch.full_like(ref3, nan))
        torch.cuda.synchronize()
        assert torch.equal(d2, ref2) and torch.equal(d1, ref1) and torch.equal(d3, ref3)
    _check_sched(plan, S, E)


@pytest.mark.parametrize("path", ["experts", "softmax_layer", "sigmoid_layer"])
def test_zero_tokens(path):
    """An empty batch (T = 0) runs through every op of the path, forward and
    backward: empty outputs and input gradients, zero weight gradients."""
    print(f"zero tokens {path}", flush=True)
    H, E, K, I = 256, 16, 4, 128
    g = torch.Generator().manual_seed(5)
    bf = torch.bfloat16
    x = torch.zeros(0, H, dtype=bf, device=DEV, requires_grad=True)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(bf).to(DEV).requires_grad_(True)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(bf).to(DEV).requires_grad_(True)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(bf).to(DEV).requires_grad_(True)
    if path == "experts":
        w = torch.zeros(0, K, device=DEV, requires_grad=True)
        out = experts_forward(x, torch.zeros(0, K, dtype=torch.int64, device=DEV), w, w1, w2)
    elif path == "softmax_layer":
        out, probs, w, idx = moe_layer(x, wr, w1, w2, K)
        assert probs.shape == (0, E) and idx.shape == (0, K)
    else:
        bias = torch.zeros(E, device=DEV)
        out, probs, w, idx = moe_layer(x, wr, w1, w2, K, router="sigmoid", expert_bias=bias,
                                       gating="hip")
    out.backward(torch.zeros(0, H, dtype=bf, device=DEV))
    torch.cuda.synchronize()
    assert out.shape == (0, H) and x.grad.shape == (0, H)
    assert not w1.grad.any() and not w2.grad.any()
    if path != "experts":
        assert wr.grad is None or not wr.grad.any()
