"""Routing against the reference's own selection ops on the device, at the
full token count of every bf16 benchmark workload.

The reference ranks with torch on the GPU: the softmax router computes
``probs = softmax(logits, dtype=float32)`` and ``torch.topk(probs, K)``
(src/models/modeling_qwen3_moe.py:269-270); the DeepSeek router
``scores = torch.sigmoid(logits)`` and ``torch.topk(scores + expert_bias, K)``
(src/models/router.py:112-127).  Those exact calls run here on the logits the
layer routes from (torch's F.linear, the reference's gating), and the HIP
router's outputs must agree:

  * every token's set of K experts is identical, hence the per-expert counts;
  * where a [T, K] position holds a different expert, the two experts' values
    are exactly equal (torch.topk's sorted output orders exact ties in an
    implementation-defined way; the kernels keep the lower id first);
  * the probabilities / scores equal torch's to fp32 rounding (the sigmoid
    scores bit for bit), and so do the renormalised weights.

The same holds on the kernel's own probabilities (torch.topk run on them),
and on the MFMA gating kernel's logits at L.
"""
from __future__ import annotations

import pytest
import torch

from moe_amd import library, ops
from moe_amd.configs import CONFIGS, make_inputs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def compare_to_topk(idx: torch.Tensor, values: torch.Tensor, K: int) -> dict:
    """idx [T,K] from the HIP router against torch.topk(values, K) on the
    same device; returns the mismatch counts (all on the device)."""
    tv, ti = torch.topk(values, K, dim=-1)
    set_diff = (idx.sort(dim=1).values != ti.sort(dim=1).values).any(dim=1)
    pos_diff = idx != ti
    ours = values.gather(1, idx)
    unequal = (pos_diff & (ours != tv)).any(dim=1)
    E = values.shape[1]
    c_ours = torch.bincount(idx.reshape(-1), minlength=E)
    c_ref = torch.bincount(ti.reshape(-1), minlength=E)
    return {"tokens_with_other_set": int(set_diff.sum()),
            "tokens_with_other_order": int((pos_diff.any(dim=1) & ~set_diff).sum()),
            "order_differences_on_unequal_values": int(unequal.sum()),
            "counts_equal": bool(torch.equal(c_ours, c_ref)),
            "_topk": (tv, ti)}


def _assert_same_routing(stats: dict, what: str):
    print(f"  {what}: other set {stats['tokens_with_other_set']}, order only "
          f"{stats['tokens_with_other_order']}, order differences on unequal values "
          f"{stats['order_differences_on_unequal_values']}, counts equal "
          f"{stats['counts_equal']}", flush=True)
    assert stats["tokens_with_other_set"] == 0, f"{what}: expert sets differ from torch.topk"
    assert stats["order_differences_on_unequal_values"] == 0, f"{what}: order differs"
    assert stats["counts_equal"], f"{what}: per-expert counts differ"


@pytest.mark.parametrize("name", ["xs_global", "m_skew", "l"])
def test_softmax_routing_matches_torch_topk(name):
    cfg = CONFIGS[name]
    print(f"softmax routing vs torch.topk: {cfg.name} T={cfg.T} E={cfg.E} K={cfg.K}", flush=True)
    inp = make_inputs(cfg, seed=0, device=DEV)
    with torch.no_grad():
        logits = library.gating_logits(inp.x, inp.w_router, "torch", fp32=False)
        assert torch.equal(logits, torch.nn.functional.linear(inp.x, inp.w_router))
        probs, w, idx = ops.router_softmax_topk(logits, cfg.K, True, inp.logit_offset)
        z = logits if inp.logit_offset is None else logits.float() + inp.logit_offset
        p_ref = torch.softmax(z, dim=-1, dtype=torch.float32)   # modeling_qwen3_moe.py:269
        torch.cuda.synchronize()
        eq = (probs == p_ref).float().mean().item()
        print(f"  probs bit-equal to torch.softmax: {eq * 100:.3f}% "
              f"(max rel diff {((probs - p_ref).abs() / p_ref).max().item():.2e})", flush=True)
        assert torch.allclose(probs, p_ref, rtol=1e-6, atol=0.0)

        st = compare_to_topk(idx, p_ref, cfg.K)              # the reference's ranking
        _assert_same_routing(st, "on torch.softmax probs")
        tv, _ = st["_topk"]
        w_ref = tv / tv.sum(dim=-1, keepdim=True)            # modeling_qwen3_moe.py:271-273
        assert torch.allclose(w, w_ref, rtol=2e-6, atol=0.0)
        _assert_same_routing(compare_to_topk(idx, probs, cfg.K), "on the kernel's probs")

        if name == "l":
            # the MFMA gating kernel's logits, and the router fused into it
            lh = library.gating_logits(inp.x, inp.w_router, "hip", fp32=False)
            _, _, ih = ops.router_softmax_topk(lh, cfg.K, True, None)
            _assert_same_routing(compare_to_topk(ih, torch.softmax(lh, -1, dtype=torch.float32),
                                                 cfg.K), "MFMA gating logits")
            pf, wf, i_f = ops.router_linear_softmax_topk(inp.x, inp.w_router, cfg.K, True)
            _assert_same_routing(compare_to_topk(i_f, torch.softmax(lh, -1, dtype=torch.float32),
                                                 cfg.K), "fused gating + router")


def test_sigmoid_routing_matches_torch_topk():
    cfg = CONFIGS["retrofit"]
    print(f"sigmoid routing vs torch.topk: {cfg.name} T={cfg.T} E={cfg.E} K={cfg.K}", flush=True)
    inp = make_inputs(cfg, seed=0, device=DEV)
    with torch.no_grad():
        logits = library.gating_logits(inp.x, inp.w_router, "torch", fp32=True)
        assert logits.dtype == torch.float32
        scores, w, idx = ops.router_sigmoid_topk(logits, inp.expert_bias, cfg.K, True, None,
                                                 None, None, torch.bfloat16)
        s_ref = torch.sigmoid(logits)                        # router.py:112
        torch.cuda.synchronize()
        neq = int((scores != s_ref).sum())
        print(f"  scores differing from torch.sigmoid: {neq} of {s_ref.numel()}", flush=True)
        assert neq == 0, "sigmoid scores differ from torch.sigmoid on the device"
        st = compare_to_topk(idx, s_ref + inp.expert_bias, cfg.K)   # router.py:115-127
        _assert_same_routing(st, "on torch.sigmoid scores + bias")
        sel = s_ref.gather(1, idx)                           # router.py:130-136, 140
        w_ref = (sel / (sel.sum(dim=-1, keepdim=True) + 1e-20)).to(torch.bfloat16)
        # the K-term fp32 sum may be taken in another order: one bf16 ulp at
        # most (the weights are positive, so their bit patterns are ordered)
        ulps = (w.view(torch.int16).int() - w_ref.view(torch.int16).int()).abs()
        print(f"  weights bit-equal: {(ulps == 0).float().mean().item() * 100:.4f}%, "
              f"max {int(ulps.max())} ulp", flush=True)
        assert int(ulps.max()) <= 1, "renormalised weights differ by more than one bf16 ulp"
