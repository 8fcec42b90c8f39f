"""Whole MoE layer (gate + experts) as one function and one module.

``moe_layer`` is the GPU form of Qwen3MoeSparseMoeBlock.forward
(src/models/modeling_qwen3_moe.py:284-289) with either router: flatten to
[T,H], gating linear, HIP router kernel, HIP expert layer.  The gating
linear's forward is torch's F.linear by default (``gating="torch"``: the very
call the reference makes, so the logits and therefore the routing are the
reference's, bit for bit) or the MFMA kernel (``gating="hip"``: the same
exact bf16 products summed in the kernel's own fp32 order, so a top-k choice
between experts whose logits tie within one bf16 rounding can differ); its
backward runs on the MFMA kernels either way.  ``gating="hip_fused"`` runs the
router (softmax, or DeepSeek sigmoid with E <= 128) in the MFMA gating kernel's
epilogue: the same bits as "hip", without the logits' round trip (shapes the
fused kernel does not cover take the two-kernel form, with the same results).
``SparseMoeBlock`` wraps it with the reference's parameter names
(``gate.weight``, ``experts.gate_up_proj``, ``experts.down_proj``).
"""
from __future__ import annotations

import torch
from torch import nn

from . import library  # registers the moe_amd:: ops
from .experts import experts_forward
from .router import gating_linear, linear_sigmoid_topk, sigmoid_topk, softmax_topk


def _fused_softmax_ok(x, w_router, gate_up_proj, down_proj) -> bool:
    E, H = w_router.shape
    return (x.is_cuda and x.dim() == 2 and x.dtype == torch.bfloat16
            and w_router.dtype == torch.bfloat16 and gate_up_proj.dtype == torch.bfloat16
            and down_proj.dtype == torch.bfloat16 and H % 256 == 0 and E % 8 == 0
            and gate_up_proj.shape[0] == E)


def moe_layer(x: torch.Tensor, w_router: torch.Tensor, gate_up_proj: torch.Tensor,
              down_proj: torch.Tensor, top_k: int, router: str = "softmax",
              renormalize: bool = True, logit_offset: torch.Tensor | None = None,
              expert_bias: torch.Tensor | None = None, scaling_factor: float | None = None,
              num_groups: int | None = None, group_topk: int | None = None,
              tokens_per_expert: torch.Tensor | None = None, gating: str = "torch"):
    """Returns (out [T,H], router_logits [T,E] fp32, weights [T,K], index [T,K])."""
    if gating not in library.GATINGS:
        raise ValueError(f"unknown gating {gating!r} (expected one of {library.GATINGS})")
    hip = gating in ("hip", "hip_fused")
    if router == "softmax" and _fused_softmax_ok(x, w_router, gate_up_proj, down_proj):
        # Gating linear + softmax router + experts as ONE autograd node (op
        # moe_amd::moe_layer_fwd), so that the two gradients of the hidden
        # states (through the gating linear and through the experts) meet
        # inside the gather backward (addend = the gating linear's dX)
        # instead of in autograd's separate add.  The arithmetic is that of
        # the composed path below: every rounding point is kept, only the
        # fp32 summation orders of the two router GEMMs differ.
        save = torch.is_grad_enabled() and any(
            t.requires_grad for t in (x, w_router, gate_up_proj, down_proj))
        res = torch.ops.moe_amd.moe_layer_fwd(x.contiguous(), w_router, gate_up_proj.contiguous(),
                                              down_proj.contiguous(), int(top_k),
                                              bool(renormalize), logit_offset, save, gating)
        return res[0], res[1], res[2], res[3]
    if router == "softmax":
        logits = gating_linear(x, w_router, fp32=False, hip=hip)
        probs, w, idx = softmax_topk(logits, top_k, renormalize, logit_offset)
    elif router == "sigmoid" and gating == "hip_fused":
        probs, w, idx = linear_sigmoid_topk(x, w_router, expert_bias, top_k, renormalize,
                                            scaling_factor, num_groups, group_topk, x.dtype,
                                            tokens_per_expert)
    elif router == "sigmoid":
        logits = gating_linear(x, w_router, fp32=True, hip=hip)
        probs, w, idx = sigmoid_topk(logits, expert_bias, top_k, renormalize, scaling_factor,
                                     num_groups, group_topk, x.dtype, tokens_per_expert)
    else:
        raise ValueError(f"unknown router {router!r}")
    out = experts_forward(x, idx, w, gate_up_proj, down_proj)
    return out, probs, w, idx


class _Gate(nn.Module):
    def __init__(self, E: int, H: int):
        super().__init__()
        self.weight = nn.Parameter(torch.zeros(E, H))


class _Bank(nn.Module):
    def __init__(self, E: int, H: int, I: int):
        super().__init__()
        self.gate_up_proj = nn.Parameter(torch.empty(E, 2 * I, H))
        self.down_proj = nn.Parameter(torch.empty(E, H, I))


class SparseMoeBlock(nn.Module):
    """Stand-alone MoE block: [B,S,H] (or [T,H]) -> same shape.  The last
    router outputs are kept in ``router_logits`` / ``topk_index``."""

    def __init__(self, hidden_size: int, num_experts: int, top_k: int, intermediate_size: int,
                 router: str = "softmax", norm_topk_prob: bool = True):
        super().__init__()
        self.top_k = top_k
        self.router = router
        self.norm_topk_prob = norm_topk_prob
        self.gate = _Gate(num_experts, hidden_size)
        self.experts = _Bank(num_experts, hidden_size, intermediate_size)
        self.logit_offset: torch.Tensor | None = None
        self.register_buffer("expert_bias", torch.zeros(num_experts, dtype=torch.float32))
        self.router_logits = None
        self.topk_index = None

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        shape = hidden_states.shape
        flat = hidden_states.reshape(-1, shape[-1])
        out, probs, _, idx = moe_layer(
            flat, self.gate.weight, self.experts.gate_up_proj, self.experts.down_proj, self.top_k,
            router=self.router, renormalize=self.norm_topk_prob, logit_offset=self.logit_offset,
            expert_bias=self.expert_bias if self.router == "sigmoid" else None)
        self.router_logits, self.topk_index = probs, idx
        return out.reshape(shape)
