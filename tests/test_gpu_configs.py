"""GPU parity of the whole layer as bench.py times it -- ``moe_layer``: gating
linear -> router kernel -> permutation -> grouped GEMMs -> combine, and the
full backward -- on each of the five benchmark workloads at their full token
count, against the CPU oracle on the same seeded inputs (configs.make_inputs:
the fixed CPU draw order, copied to the device), with both gating sources
(torch's F.linear and the MFMA gating kernel; at L and XS-global also the
router fused into the gating kernel's epilogue).

Per workload and gating source:
  * routing, every token: with the logits the layer used (recomputed by the
    same deterministic call), the indices and the counts equal the oracle's
    bit for bit (softmax router); for the DeepSeek router the scores equal
    torch.sigmoid's on the device bit for bit, and the indices equal the
    oracle's selection on them (tests/test_gpu_routing_torch.py compares
    with torch.topk itself);
  * output and d_x (experts' and router's parts together, so the router part
    carries the routing-weight gradient) of a 256-token sample, recomputed by
    the oracle from those tokens; d_topk_weights itself, which the one-node
    layer keeps internal, on M's skewed routing through the expert-layer op
    (test_layer_routing_weight_grad_sampled);
  * d_gate_up_proj / d_down_proj of the most- and least-loaded experts from
    all their routed rows (each expert's weight gradient depends on its own
    rows only); experts that received no token have exactly zero gradients;
  * the router weight gradient end to end on a token chunk (the layer run on
    the chunk alone; the whole batch for XS-global), against the oracle's
    full chain: router -> experts -> expert backward -> router backward ->
    d_logits^T x.

Tolerance: max |gpu - oracle| / max |oracle| <= 2e-2 per bf16 tensor (the
north-star bound); 1e-5 for the fp32 XS-standard layer against the fp64
eager oracle.  The oracle is handed only the experts that the checked tokens
touch (re-indexed), which keeps the 1792-expert bank off the host.
"""
from __future__ import annotations

import pytest
import torch

from moe_amd import library, ops
from moe_amd.configs import CONFIGS, make_inputs
from moe_amd.layer import moe_layer
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2e-2
SAMPLE = 256


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


_CACHE: dict = {}


def _inputs(name):
    """Seeded full-size inputs of a workload on the GPU (cached: the
    1792-expert bank takes a while to draw on the CPU)."""
    if name not in _CACHE:
        _CACHE.clear()  # one workload's inputs resident at a time
        torch.cuda.empty_cache()
        print(f"[inputs] {name}: drawing on the CPU in the fixed draw order", flush=True)
        _CACHE[name] = make_inputs(CONFIGS[name], seed=0, device=DEV)
    return _CACHE[name]


def _compact(idx, w1, w2, E):
    """(idx re-indexed onto the experts it uses, their gate_up/down weights on
    the CPU).  Ids outside [0,E) stay sentinels (mapped to len(used))."""
    flat = idx.reshape(-1)
    used = torch.unique(flat[(flat >= 0) & (flat < E)])
    remap = torch.full((E + 1,), len(used), dtype=torch.int64)
    remap[used] = torch.arange(len(used))
    sub = remap[flat.clamp(0, E)].view(idx.shape)
    return sub, w1[used.to(w1.device)].cpu(), w2[used.to(w2.device)].cpu(), used


def _run_layer(cfg, inp, x, gating, need_wr=True):
    """moe_layer fwd+bwd with fresh leaves; returns (out, probs, w, idx, grads)."""
    xl = x.detach().clone().requires_grad_(True)
    wr = inp.w_router.detach().clone().requires_grad_(need_wr)
    w1 = inp.gate_up_proj.requires_grad_(True)
    w2 = inp.down_proj.requires_grad_(True)
    w1.grad = w2.grad = None
    out, probs, w, idx = moe_layer(xl, wr, w1, w2, cfg.K, router=cfg.router,
                                   logit_offset=inp.logit_offset, expert_bias=inp.expert_bias,
                                   gating=gating)
    return out, probs, w, idx, xl, wr, w1, w2


def _logits(cfg, inp, x, gating):
    """The logits the layer computed (every gating source is deterministic)."""
    with torch.no_grad():
        return library.gating_logits(x, inp.w_router, gating, fp32=cfg.router == "sigmoid")


def _check_routing(cfg, inp, logits, probs, w, idx):
    """Full-batch routing check; returns the oracle's (probs, weights, idx)."""
    lc = logits.cpu()
    if cfg.router == "softmax":
        off = None if inp.logit_offset is None else inp.logit_offset.cpu()
        p_ref, w_ref, i_ref = O.softmax_router(lc, cfg.K, True, off)
        assert torch.equal(idx.cpu(), i_ref), "routing indices differ from the oracle"
        assert torch.allclose(probs.cpu(), p_ref, rtol=1e-5, atol=1e-7)
        assert torch.allclose(w.cpu(), w_ref, rtol=1e-5, atol=1e-7)
        return p_ref, w_ref, i_ref
    bias = inp.expert_bias.cpu()
    # The scores are the reference's own: torch.sigmoid on this device
    # (router.py:112), bit for bit; the oracle then routes from them.
    s_gpu = torch.sigmoid(logits)
    assert torch.equal(probs, s_gpu), "sigmoid scores differ from torch.sigmoid on the GPU"
    sc = s_gpu.cpu()
    w_ref, i_ref = O.sigmoid_router_from_scores(sc, bias, cfg.K, True, None, None, None,
                                                torch.float32)
    assert torch.equal(idx.cpu(), i_ref), "selection differs from the oracle's"
    s_cpu = torch.sigmoid(lc.float())  # the oracle's CPU sigmoid: within fp32 rounding
    assert torch.allclose(sc, s_cpu, rtol=2e-6, atol=1e-7)
    # weights: the selected scores renormalised (+1e-20), rounded to bf16 once
    assert _rel(w, w_ref.to(w.dtype)) < 8e-3
    return sc, w_ref, i_ref


def _oracle_tokens(cfg, inp, toks, idx, w, probs_ref):
    """Oracle forward/backward of the tokens `toks` under the layer's routing
    (idx, w): (out, d_x incl. the router part, d_topk_weights)."""
    E = cfg.E
    xs = inp.x[toks].cpu()
    ws = w[toks].detach().cpu()
    sub, w1c, w2c, _ = _compact(idx[toks].cpu(), inp.gate_up_proj.detach(),
                                inp.down_proj.detach(), E)
    out_ref, cache = O.experts_forward(xs, sub, ws, w1c, w2c)
    dx_e, dw_ref, _, _, _ = O.experts_backward(cache, xs, ws, w1c, w2c, inp.dout[toks].cpu())
    wr = inp.w_router.cpu().float()
    ic = idx[toks].cpu()
    if cfg.router == "softmax":
        dl = O.softmax_router_backward(probs_ref[toks], ic, dw_ref, None, True, torch.bfloat16)
        dx_r = (dl.float() @ wr).to(torch.bfloat16)
    else:
        dl = O.sigmoid_router_backward(probs_ref[toks], ic, dw_ref, None, True, None)
        dx_r = (dl @ wr).to(torch.bfloat16)
    dx = (dx_e.float() + dx_r.float()).to(torch.bfloat16)
    return out_ref, dx, dw_ref


def _expert_dw(cfg, inp, idx, w, e):
    """Oracle d_gate_up_proj[e], d_down_proj[e] from every row routed to e."""
    rows = (idx == e).any(-1).nonzero().flatten()
    toks = rows.cpu()
    ie = idx[rows].cpu()
    sub = torch.where(ie == e, torch.zeros_like(ie), torch.ones_like(ie))  # 1 = sentinel
    xs, ws = inp.x[rows].cpu(), w[rows].detach().cpu()
    w1c = inp.gate_up_proj.detach()[e:e + 1].cpu()
    w2c = inp.down_proj.detach()[e:e + 1].cpu()
    _, cache = O.experts_forward(xs, sub, ws, w1c, w2c)
    _, _, dw1, dw2, _ = O.experts_backward(cache, xs, ws, w1c, w2c, inp.dout[rows].cpu())
    return dw1[0], dw2[0], toks.numel()


def _chunk_router_grad(cfg, inp, gating, T_chunk):
    """d_w_router and d_x of the layer run on the first T_chunk tokens alone,
    against the oracle's full chain on the same tokens."""
    x = inp.x[:T_chunk]
    out, probs, w, idx, xl, wr, w1, w2 = _run_layer(cfg, inp, x, gating)
    out.backward(inp.dout[:T_chunk])
    torch.cuda.synchronize()
    logits = _logits(cfg, inp, x, gating)
    p_ref, _, _ = _check_routing(cfg, inp, logits, probs, w, idx)
    toks = torch.arange(T_chunk)
    out_ref, dx_ref, dw_ref = _oracle_tokens(cfg, inp, toks, idx, w, p_ref)
    # router weight gradient: d_logits^T x over the chunk (fp32 products, one bf16 rounding)
    ic = idx.cpu()
    if cfg.router == "softmax":
        dl = O.softmax_router_backward(p_ref, ic, dw_ref, None, True, torch.bfloat16).float()
    else:
        dl = O.sigmoid_router_backward(p_ref, ic, dw_ref, None, True, None)
    dwr_ref = (dl.t().double() @ x.cpu().double()).to(torch.bfloat16)
    e_out, e_dx, e_wr = _rel(out.detach(), out_ref), _rel(xl.grad, dx_ref), _rel(wr.grad, dwr_ref)
    print(f"  chunk T={T_chunk}: out {e_out:.2e}  d_x {e_dx:.2e}  d_w_router {e_wr:.2e}",
          flush=True)
    assert e_out < TOL and e_dx < TOL and e_wr < TOL


def test_layer_routing_weight_grad_sampled():
    """d_topk_weights of the one-node softmax layer is internal to the op;
    the expert-layer op exposes it: on the M workload's routing (skewed),
    the weight gradient of a token sample against the oracle."""
    from moe_amd.experts import experts_forward
    cfg = CONFIGS["m_skew"]
    inp = _inputs("m_skew")
    logits = _logits(cfg, inp, inp.x, "torch")
    probs, w, idx = ops.router_softmax_topk(logits, cfg.K, True, inp.logit_offset)
    wl = w.detach().clone().requires_grad_(True)
    out = experts_forward(inp.x, idx, wl, inp.gate_up_proj.detach(), inp.down_proj.detach())
    out.backward(inp.dout)
    torch.cuda.synchronize()
    p_ref, w_ref, i_ref = O.softmax_router(logits.cpu(), cfg.K, True, inp.logit_offset.cpu())
    assert torch.equal(idx.cpu(), i_ref)
    toks = torch.randperm(cfg.T, generator=torch.Generator().manual_seed(2))[:SAMPLE]
    _, _, dw_ref = _oracle_tokens(cfg, inp, toks, idx, w, p_ref)
    err = _rel(wl.grad[toks], dw_ref)
    print(f"M d_topk_weights sample: {err:.2e}", flush=True)
    assert err < TOL


# M first: the sampled routing-weight test above drew its inputs (one
# workload is cached at a time); Retrofit last, for the schedule test below.
BF16_CASES = ([(c, g) for c in ("m_skew", "xs_global", "l", "retrofit") for g in ("torch", "hip")]
              + [("l", "hip_fused"), ("xs_global", "hip_fused")])


@pytest.mark.parametrize("name,gating", BF16_CASES)
def test_layer_config_parity(name, gating):
    cfg = CONFIGS[name]
    print(f"layer parity {cfg.name} (T={cfg.T} H={cfg.H} E={cfg.E} K={cfg.K}) "
          f"gating={gating}", flush=True)
    inp = _inputs(name)
    out, probs, w, idx, xl, wr, w1, w2 = _run_layer(cfg, inp, inp.x, gating)
    out.backward(inp.dout)
    torch.cuda.synchronize()
    print("  fwd+bwd done", flush=True)

    logits = _logits(cfg, inp, inp.x, gating)
    p_ref, _, _ = _check_routing(cfg, inp, logits, probs, w, idx)
    counts = torch.bincount(idx.reshape(-1), minlength=cfg.E).cpu()
    imb = counts.max().item() / (cfg.S / cfg.E)
    print(f"  routing ok; load imbalance max/mean {imb:.2f}, empty experts "
          f"{int((counts == 0).sum())}", flush=True)

    g = torch.Generator().manual_seed(1)
    toks = torch.randperm(cfg.T, generator=g)[:SAMPLE]
    out_ref, dx_ref, dw_ref = _oracle_tokens(cfg, inp, toks, idx, w, p_ref)
    e_out = _rel(out.detach()[toks], out_ref)
    e_dx = _rel(xl.grad[toks], dx_ref)
    print(f"  sample: out {e_out:.2e}  d_x {e_dx:.2e}", flush=True)
    assert e_out < TOL and e_dx < TOL

    nz = counts.clone()
    nz[nz == 0] = counts.max() + 1
    for e in (int(counts.argmax()), int(nz.argmin())):
        dw1, dw2, n = _expert_dw(cfg, inp, idx, w, e)
        e1, e2 = _rel(w1.grad[e], dw1), _rel(w2.grad[e], dw2)
        print(f"  expert {e} ({n} tokens): dW1 {e1:.2e}  dW2 {e2:.2e}", flush=True)
        assert e1 < TOL and e2 < TOL
    for e in (counts == 0).nonzero().flatten().tolist()[:8]:
        assert not w1.grad[e].any() and not w2.grad[e].any(), f"untouched expert {e}"

    T_chunk = cfg.T if name == "xs_global" else (32 if cfg.E > 256 else 2048)
    _chunk_router_grad(cfg, inp, gating, T_chunk)
    del out, probs, w, idx, xl, wr
    w1.grad = w2.grad = None


def test_retrofit_dw_schedule_at_1792_experts():
    """The dW GEMMs' claimed-tile schedule at the Retrofit bank (E = 1792,
    Retrofit routing): the three dW GEMMs, writing into NaN-filled outputs,
    bit-identical to the static walk on two launches in a row (the 1437 or so
    experts without rows included), and the schedule tables well-formed;
    then the two accumulating forms (fused gradient accumulation into the
    bank's main_grad) at the full bank: acc += dW bit for bit as torch's bf16
    add gives it, the experts without rows (NaN-filled) untouched."""
    from test_gpu_experts import _check_sched
    cfg = CONFIGS["retrofit"]
    inp = _inputs("retrofit")
    logits = _logits(cfg, inp, inp.x, "torch")
    _, _, idx = ops.router_sigmoid_topk(logits, inp.expert_bias, cfg.K, True, None, None, None,
                                        torch.bfloat16)
    E, S, H, I = cfg.E, cfg.S, cfg.H, cfg.I
    plan = ops.permute(idx, E)
    g = torch.Generator(device=DEV).manual_seed(3)
    dgu = torch.randn(S, 2 * I, generator=g, device=DEV).to(torch.bfloat16)
    dy = torch.randn(S, H, generator=g, device=DEV).to(torch.bfloat16)
    act = torch.randn(S, I, generator=g, device=DEV).to(torch.bfloat16)
    dout = torch.randn(cfg.T, H, generator=g, device=DEV).to(torch.bfloat16)
    ref1 = ops.gemm_gate_up_backward_dw(dgu, inp.x, plan, (E, 2 * I, H), scheduled=False)
    ref2 = ops.gemm_down_backward_dw(dy, act, plan, (E, H, I), scheduled=False)
    ref3 = ops.gemm_down_backward_dw_gathered(dout, act, plan, (E, H, I), scheduled=False)
    nan = float("nan")
    for rep in range(2):
        # NaN-filled outputs: every tile is written, the zero tiles included
        d1 = ops.gemm_gate_up_backward_dw(dgu, inp.x, plan, (E, 2 * I, H),
                                          out=torch.full_like(ref1, nan))
        d2 = ops.gemm_down_backward_dw(dy, act, plan, (E, H, I), out=torch.full_like(ref2, nan))
        d3 = ops.gemm_down_backward_dw_gathered(dout, act, plan, (E, H, I),
                                                out=torch.full_like(ref3, nan))
        torch.cuda.synchronize()
        assert torch.equal(d1, ref1) and torch.equal(d2, ref2), f"launch {rep}"
        assert torch.equal(d3, ref3), f"launch {rep}"
        del d1, d2, d3
    load = _check_sched(plan, S, E)
    print(f"retrofit per-XCD rows {load}", flush=True)
    empty = plan.counts == 0
    for ref, fn, args in ((ref1, ops.gemm_gate_up_backward_dw_accumulate, (dgu, inp.x, plan)),
                          (ref3, ops.gemm_down_backward_dw_gathered_accumulate,
                           (dout, act, plan))):
        acc = torch.randn(ref.shape, generator=g, device=DEV).to(torch.bfloat16)
        acc[empty] = nan
        exp = acc.clone()
        exp[~empty] += ref[~empty]
        fn(*args, acc)
        torch.cuda.synchronize()
        assert torch.equal(acc.view(torch.int16), exp.view(torch.int16)), fn.__name__
        del acc, exp
    print("retrofit accumulating dW GEMMs ok", flush=True)


def test_xs_standard_fp32_layer():
    """XS standard (fp32, T = 2048, H = 1024, E = 16, K = 4): the fp32 grouped
    GEMMs (v_mfma_f32_32x32x2_f32) through moe_layer with torch's fp32
    gating: routing bit-exact; the forward (the config's pass) and, beyond
    it, every gradient within 1e-5 of the fp64 eager oracle (the reference's
    eager experts loop, modeling_qwen3_moe.py:230-254, in float64)."""
    cfg = CONFIGS["xs_std"]
    print(f"XS standard fp32 T={cfg.T} H={cfg.H} E={cfg.E} K={cfg.K}", flush=True)
    inp = make_inputs(cfg, seed=0, device=DEV)
    assert inp.x.dtype == torch.float32
    out, probs, w, idx, xl, wr, w1, w2 = _run_layer(cfg, inp, inp.x, "torch")
    out.backward(inp.dout)
    torch.cuda.synchronize()
    logits = _logits(cfg, inp, inp.x, "torch")
    _check_routing(cfg, inp, logits, probs, w, idx)
    # fp64 oracle: the eager loop and its autograd, on the same routing
    f64 = [t.detach().cpu().double().requires_grad_(True)
           for t in (inp.x, w, inp.gate_up_proj, inp.down_proj)]
    ref = O.experts_eager(f64[0], idx.cpu(), f64[1], f64[2], f64[3])
    grads = torch.autograd.grad(ref, f64, inp.dout.cpu().double())
    # the router part of d_x and d_w_router (fp64 chain through the softmax)
    p64 = torch.softmax(logits.cpu().double(), -1)
    dl = O.softmax_router_backward(p64, idx.cpu(), grads[1], None, True, torch.float64)
    dx_ref = grads[0] + dl @ inp.w_router.cpu().double()
    dwr_ref = dl.t() @ inp.x.cpu().double()
    errs = {"out": _rel(out.detach(), ref.detach()), "d_x": _rel(xl.grad, dx_ref),
            "d_w_router": _rel(wr.grad, dwr_ref), "d_gate_up_proj": _rel(w1.grad, grads[2]),
            "d_down_proj": _rel(w2.grad, grads[3])}
    print("  " + "  ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    assert all(v <= 1e-5 for v in errs.values()), errs
