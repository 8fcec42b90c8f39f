"""Every tensor of one L step (T=65536, H=2048, E=128, K=8, I=768, the
headline workload) against the CPU oracle, not a sample: the layer as
bench.py times it (torch's gating linear -> HIP router -> permutation ->
grouped GEMMs -> combine, then the whole backward) and the oracle's forward
and backward on the same routing, over all 65,536 tokens and all 128
experts.

Per tensor: max |gpu - oracle| / max |oracle| <= 2e-2 (the north-star bf16
bound) -- for out and d_x over the whole batch and in every block of 4,096
tokens, for d_gate_up_proj and d_down_proj per expert (each expert's
gradient normalised by its own largest entry), and for d_w_router.
"""
from __future__ import annotations

import pytest
import torch

from moe_amd import library
from moe_amd.configs import CONFIGS, make_inputs
from moe_amd.layer import moe_layer
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2e-2


def _rel_rows(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Per leading index: max |a - b| / max |b| over the remaining dims."""
    a, b = a.float().flatten(1), b.float().flatten(1)
    return (a - b).abs().amax(1) / b.abs().amax(1).clamp_min(1e-30)


def test_l_step_every_tensor_against_oracle():
    cfg = CONFIGS["l"]
    print(f"full-tensor L: T={cfg.T} H={cfg.H} E={cfg.E} K={cfg.K} I={cfg.I}", flush=True)
    inp = make_inputs(cfg, seed=0, device=DEV)
    x = inp.x.clone().requires_grad_(True)
    wr = inp.w_router.clone().requires_grad_(True)
    w1 = inp.gate_up_proj.requires_grad_(True)
    w2 = inp.down_proj.requires_grad_(True)
    out, probs, w, idx = moe_layer(x, wr, w1, w2, cfg.K, gating="torch")
    out.backward(inp.dout)
    torch.cuda.synchronize()
    print("  GPU fwd+bwd done", flush=True)
    with torch.no_grad():
        logits = library.gating_logits(inp.x, inp.w_router, "torch", fp32=False).cpu()

    p_ref, w_ref, i_ref = O.softmax_router(logits, cfg.K, True)
    assert torch.equal(idx.cpu(), i_ref)
    xc, w1c, w2c = inp.x.cpu(), inp.gate_up_proj.detach().cpu(), inp.down_proj.detach().cpu()
    out_ref, cache = O.experts_forward(xc, i_ref, w_ref, w1c, w2c)
    dx_e, dw_ref, dw1_ref, dw2_ref, _ = O.experts_backward(cache, xc, w_ref, w1c, w2c,
                                                           inp.dout.cpu())
    del cache
    dl = O.softmax_router_backward(p_ref, i_ref, dw_ref, None, True, torch.bfloat16).float()
    dx_ref = (dx_e.float() + (dl @ inp.w_router.cpu().float()).to(torch.bfloat16).float()
              ).to(torch.bfloat16)
    dwr_ref = (dl.t().double() @ xc.double()).to(torch.bfloat16)
    print("  oracle fwd+bwd done", flush=True)

    blocks = cfg.T // 4096
    checks = {
        "out": _rel_rows(out.detach().cpu().view(blocks, -1), out_ref.view(blocks, -1)),
        "d_x": _rel_rows(x.grad.cpu().view(blocks, -1), dx_ref.view(blocks, -1)),
        "d_gate_up_proj": _rel_rows(w1.grad.cpu(), dw1_ref),
        "d_down_proj": _rel_rows(w2.grad.cpu(), dw2_ref),
        "d_w_router": _rel_rows(wr.grad.cpu().view(1, -1), dwr_ref.view(1, -1)),
    }
    whole = {"out": (out.detach().cpu(), out_ref), "d_x": (x.grad.cpu(), dx_ref)}
    for k, (a, b) in whole.items():
        print(f"  {k}: whole batch {_rel_rows(a.view(1, -1), b.view(1, -1)).item():.2e}",
              flush=True)
    for k, v in checks.items():
        print(f"  {k}: worst of {v.numel()} {v.max().item():.2e} (median "
              f"{v.median().item():.2e})", flush=True)
    bad = {k: v.max().item() for k, v in checks.items() if not (v <= TOL).all()}
    assert not bad, bad
    w1.grad = w2.grad = None
