"""Whole MoE layer (gate + experts) as one function and one module.

``moe_layer`` is the GPU form of Qwen3MoeSparseMoeBlock.forward
(src/models/modeling_qwen3_moe.py:284-289) with either router: flatten to
[T,H], gating linear (MFMA kernel for bf16; ``gating="torch"`` keeps F.linear),
HIP router kernel, HIP expert layer.
``SparseMoeBlock`` wraps it with the reference's parameter names
(``gate.weight``, ``experts.gate_up_proj``, ``experts.down_proj``).
"""
from __future__ import annotations

import torch
from torch import nn

from . import ops
from .experts import experts_forward
from .router import SigmoidTopKFunction, SoftmaxTopKFunction, gating_linear


class SoftmaxMoELayerFunction(torch.autograd.Function):
    """Gating linear + softmax router + experts as ONE autograd node, so that
    the two gradients of the hidden states (through the gating linear and
    through the experts) meet inside the gather backward
    (``gather_backward(..., addend=router dx)``) instead of in autograd's
    separate add, and the gating linear's dX runs on the MFMA kernel.  The
    arithmetic is that of the composed path (RouterLinearFunction,
    SoftmaxTopKFunction, MoEExpertsFunction): every rounding point is kept,
    only the fp32 summation orders of the two router GEMMs differ.

    Inputs: x [T,H] bf16, w_router [E,H] bf16, gate_up_proj, down_proj (bf16).
    Outputs: (out [T,H], probs [T,E] fp32, weights [T,K] fp32, index [T,K])."""

    @staticmethod
    def forward(ctx, x, w_router, gate_up_proj, down_proj, top_k, renormalize, logit_offset):
        ctx.set_materialize_grads(False)
        logits = ops.router_linear(x, w_router, torch.bfloat16)
        probs, w, idx = ops.router_softmax_topk(logits, top_k, renormalize, logit_offset)
        del logits
        plan = ops.permute(idx, gate_up_proj.shape[0])
        need = any(ctx.needs_input_grad)
        gu, act = ops.gemm_gate_up_swiglu(x, plan, gate_up_proj, save_gate_up=need)
        y = ops.gemm_down(act, plan, down_proj)
        out = ops.combine(y, plan, w)
        ctx.mark_non_differentiable(idx)
        if need:
            # y and act are not kept: the backward recomputes act from gu
            ctx.save_for_backward(x, w_router, gate_up_proj, down_proj, gu, probs, w, idx)
            ctx.plan = plan
            ctx.renormalize = renormalize
        return out, probs, w, idx

    @staticmethod
    def backward(ctx, d_out, d_probs, d_w, d_idx):
        x, w_router, gate_up_proj, down_proj, gu, probs, w, idx = ctx.saved_tensors
        plan = ctx.plan
        need_x, need_wr, need_w1, need_w2 = ctx.needs_input_grad[:4]
        if d_out is None:
            d_out = torch.zeros(x.shape, dtype=x.dtype, device=x.device)
        d_out = d_out.to(x.dtype)
        # combine backward fused into GEMM-2's backward (no [S,H] d_y)
        d_gu, act_w, dw = ops.gemm_down_backward_fused(d_out, plan, down_proj, gu, w)
        d_w2 = (ops.gemm_down_backward_dw_gathered(d_out, act_w, plan, down_proj.shape)
                if need_w2 else None)
        del act_w
        d_w1 = (ops.gemm_gate_up_backward_dw(d_gu, x, plan, gate_up_proj.shape)
                if need_w1 else None)
        if d_w is not None:
            dw = dw + d_w.float()
        d_logits = ops.router_softmax_topk_backward(probs, idx, dw, d_probs, ctx.renormalize,
                                                    torch.bfloat16)
        d_wr = None
        if need_wr:
            if w_router.shape[0] <= 256:
                d_wr = ops.router_linear_backward_dw(d_logits, x)
            else:
                d_wr = d_logits.t().contiguous() @ x
        d_x = None
        if need_x:
            d_xs = ops.gemm_gate_up_backward_dx(d_gu, plan, gate_up_proj)
            d_x = ops.gather_backward(d_xs, plan,
                                      addend=ops.router_linear_backward_dx(d_logits, w_router))
        ctx.plan = None
        return d_x, d_wr, d_w1, d_w2, None, None, None


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
              tokens_per_expert: torch.Tensor | None = None, gating: str = "hip"):
    """Returns (out [T,H], router_logits [T,E] fp32, weights [T,K], index [T,K])."""
    if gating not in ("hip", "torch"):
        raise ValueError(f"unknown gating {gating!r}")
    hip = gating == "hip"
    if router == "softmax" and hip and _fused_softmax_ok(x, w_router, gate_up_proj, down_proj):
        return SoftmaxMoELayerFunction.apply(x.contiguous(), w_router, gate_up_proj.contiguous(),
                                             down_proj.contiguous(), top_k, renormalize,
                                             logit_offset)
    if router == "softmax":
        logits = gating_linear(x, w_router, fp32=False, hip=hip)
        probs, w, idx = SoftmaxTopKFunction.apply(logits, top_k, renormalize, logit_offset)
    elif router == "sigmoid":
        logits = gating_linear(x, w_router, fp32=True, hip=hip)
        probs, w, idx = SigmoidTopKFunction.apply(logits, expert_bias, top_k, renormalize,
                                                  scaling_factor, num_groups, group_topk,
                                                  x.dtype, tokens_per_expert)
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
