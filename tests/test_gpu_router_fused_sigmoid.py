"""The DeepSeek-V3 router fused into the gating linear's epilogue
(moe_amd_router_linear_sigmoid_topk) on the GPU.

Per case, against the two-kernel form on the same device -- router_linear
(fp32 logits) followed by router_sigmoid_topk -- bit for bit: the fp32
logits it writes, the sigmoid scores, the weights, the ids and the selection
counts; the scores against torch.sigmoid on the device bit for bit (the
reference's call, src/models/router.py:112); the ids and weights against the
oracle's selection on those scores (router.py:22-70, :115-140).  Shapes: the
reference's DeepSeek configurations (configs/scaling/l_deepseek_standard.yaml:
E=64, K=8, 8 groups keep 4, scaling 2.5; xs_deepseek_standard / debug8 e16 /
e16_k1 / e64), flat top-K, ragged T and fewer tokens than one tile.  Then the
op's gradients and the whole layer with gating="hip_fused" against
gating="hip" bit for bit.
"""
from __future__ import annotations

import pytest
import torch

from moe_amd import ops
from moe_amd.layer import moe_layer
from moe_amd.router import MI355XDeepSeekRouter, gating_linear, linear_sigmoid_topk, sigmoid_topk
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16) if t.dtype == torch.bfloat16 else t.view(torch.int32)


@pytest.mark.parametrize("T,H,E,K,groups,gtk,sf,wdt", [
    (65536, 2048, 64, 8, 8, 4, 2.5, torch.bfloat16),   # L DeepSeek standard, full T
    (16384, 1024, 16, 4, 8, 4, None, torch.bfloat16),  # XS DeepSeek standard
    (4096, 512, 16, 1, 8, 1, None, torch.float32),     # e16, top-1, one group kept
    (2048, 1024, 64, 4, 8, 4, None, torch.float32),    # e64
    (1000, 256, 128, 8, None, None, None, torch.float32),  # flat, 16 experts per lane
    (777, 128, 72, 6, None, None, 1.5, torch.bfloat16),    # flat, ragged E and T
    (333, 192, 128, 8, 8, 2, None, torch.bfloat16),    # groups of 16 (one lane each)
    (5, 64, 32, 4, 4, 2, 1.5, torch.bfloat16),         # fewer tokens than one tile
])
def test_fused_sigmoid_router_parity(T, H, E, K, groups, gtk, sf, wdt):
    print(f"fused sigmoid router T={T} H={H} E={E} K={K} groups={groups}/{gtk} sf={sf} {wdt}",
          flush=True)
    g = torch.Generator().manual_seed(T + E + K)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    bias = ((torch.rand(E, generator=g) * 2 - 1) * 0.5).to(DEV)
    for renorm in (True, False):
        tpe1 = torch.zeros(E, device=DEV)
        tpe2 = torch.zeros(E, device=DEV)
        sc, w, idx, lg = ops.router_linear_sigmoid_topk(x, wr, bias, K, renorm, sf, groups, gtk,
                                                        wdt, tpe1, return_logits=True)
        logits = ops.router_linear(x, wr, torch.float32)
        s2, w2, i2 = ops.router_sigmoid_topk(logits, bias, K, renorm, sf, groups, gtk, wdt, tpe2)
        s3, w3, i3 = ops.router_linear_sigmoid_topk(x, wr, bias, K, renorm, sf, groups, gtk, wdt)
        torch.cuda.synchronize()
        assert torch.equal(_bits(lg), _bits(logits)), "fused logits differ from router_linear's"
        assert torch.equal(idx, i2) and torch.equal(i3, i2), "fused routing ids differ"
        for a, b in ((sc, s2), (w, w2), (s3, s2), (w3, w2)):
            assert torch.equal(_bits(a), _bits(b)), "fused values differ"
        assert torch.equal(tpe1, tpe2), "selection counts differ"
        assert torch.equal(_bits(sc), _bits(torch.sigmoid(lg))), "scores differ from torch.sigmoid"
        if T <= 20000:
            w_ref, i_ref = O.sigmoid_router_from_scores(sc.cpu(), bias.cpu(), K, renorm, sf,
                                                        groups, gtk, wdt)
            assert torch.equal(idx.cpu(), i_ref), "selection differs from the oracle's"
            assert torch.allclose(w.cpu().float(), w_ref.float(),
                                  rtol=1e-5 if wdt == torch.float32 else 8e-3, atol=1e-7)
        counts = torch.bincount(idx.reshape(-1), minlength=E).float()
        assert torch.equal(tpe1, counts)


def test_fused_sigmoid_router_gradients_and_module():
    """The op's gradients (sigmoid_topk backward into the fp32 gating
    linear's gradients) equal those of the two-op form bit for bit; the
    router module with fused_router = True gives the unfused module's
    outputs, counts and gradients."""
    T, H, E, K = 3000, 512, 64, 8
    g = torch.Generator().manual_seed(11)
    x0 = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    w0 = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    bias = ((torch.rand(E, generator=g) * 2 - 1) * 0.5).to(DEV)
    dsc = torch.randn(T, E, generator=g).to(DEV)
    dw_ = torch.randn(T, K, generator=g).to(DEV)

    def run(fused):
        x = x0.clone().requires_grad_(True)
        wr = w0.clone().requires_grad_(True)
        if fused:
            sc, w, idx = linear_sigmoid_topk(x, wr, bias, K, True, 2.5, 8, 4, torch.float32)
        else:
            sc, w, idx = sigmoid_topk(gating_linear(x, wr, fp32=True, hip=True), bias, K, True,
                                      2.5, 8, 4, torch.float32)
        torch.autograd.backward((sc, w), (dsc, dw_))
        return sc.detach(), w.detach(), idx, x.grad, wr.grad

    for a, b in zip(run(True), run(False)):
        assert torch.equal(a, b)

    from transformers import Qwen3MoeConfig
    cfg = Qwen3MoeConfig(hidden_size=H, num_experts=E, num_experts_per_tok=K,
                         norm_topk_prob=True)
    cfg.topk_scaling_factor, cfg.num_groups, cfg.group_topk = 2.5, 8, 4
    outs = []
    for fused in (True, False):
        r = MI355XDeepSeekRouter(cfg).to(DEV)
        r.fused_router = fused
        r.hip_gating_linear = True
        r.weight = torch.nn.Parameter(w0.clone())  # bf16, as the bf16 model holds it
        with torch.no_grad():
            r.expert_bias.copy_(bias)
        xi = x0.clone().requires_grad_(True)
        sc, w, idx = r(xi)
        (sc.float().sum() + w.float().square().sum()).backward()
        outs.append((sc.detach(), w.detach(), idx, r.local_tokens_per_expert.clone(),
                     r._last_top_k_idx, xi.grad, r.weight.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_layer_deepseek_hip_fused_matches_hip():
    """moe_layer with the DeepSeek router: gating="hip_fused" (router in the
    gating kernel) against gating="hip" (gating kernel, then router kernel):
    output, routing, counts and every gradient bit for bit."""
    T, H, E, K, I = 4096, 1024, 64, 8, 256
    g = torch.Generator().manual_seed(3)
    x0 = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    wr0 = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    w10 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    w20 = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    bias = ((torch.rand(E, generator=g) * 2 - 1) * 0.5).to(DEV)
    dout = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    res = []
    for gating in ("hip_fused", "hip"):
        leaves = [t.clone().requires_grad_(True) for t in (x0, wr0, w10, w20)]
        tpe = torch.zeros(E, device=DEV)
        out, sc, w, idx = moe_layer(*leaves, K, router="sigmoid", expert_bias=bias,
                                    scaling_factor=2.5, num_groups=8, group_topk=4,
                                    tokens_per_expert=tpe, gating=gating)
        grads = torch.autograd.grad(out, leaves, dout)
        torch.cuda.synchronize()
        res.append((out, sc, w, idx, tpe) + tuple(grads))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_fused_sigmoid_router_rejects():
    """Shapes outside the fused kernel's are refused with the two-kernel form
    named."""
    H = 128
    x = torch.zeros(64, H, dtype=torch.bfloat16, device=DEV)
    for E, K, groups, gtk in ((136, 8, None, None), (64, 9, None, None), (128, 8, 16, 4),
                              (64, 8, 8, 3)):
        wr = torch.zeros(E, H, dtype=torch.bfloat16, device=DEV)
        with pytest.raises(RuntimeError, match="router_linear_sigmoid_topk"):
            ops.router_linear_sigmoid_topk(x, wr, None, K, True, None, groups, gtk)
