"""The expert layer: permute -> grouped GEMM-1 + SwiGLU -> grouped GEMM-2 ->
combine, with a hand-written backward, all on the HIP kernels.

``experts_forward`` is the functional form; ``mi355x_experts_forward`` has
the transformers ExpertsInterface signature
``fn(self, hidden_states [T,H], top_k_index [T,K], top_k_weights [T,K])``
(transformers/integrations/moe.py:377-382) and reads the bank's
``gate_up_proj [E,2I,H]`` / ``down_proj [E,H,I]`` from ``self``.
"""
from __future__ import annotations

import torch

from . import ops


class MoEExpertsFunction(torch.autograd.Function):
    """Autograd node of one expert-layer call.

    Differentiable w.r.t. hidden_states, top_k_weights, gate_up_proj and
    down_proj (not top_k_index), as the reference's grouped_mm path is
    (transformers/integrations/moe.py:377-478; backward formulas :226-242)."""

    @staticmethod
    def forward(ctx, hidden_states, top_k_index, top_k_weights, gate_up_proj, down_proj):
        E = gate_up_proj.shape[0]
        plan = ops.permute(top_k_index, E)
        need_grad = any(ctx.needs_input_grad)
        gu, act = ops.gemm_gate_up_swiglu(hidden_states, plan, gate_up_proj,
                                          save_gate_up=need_grad)
        y = ops.gemm_down(act, plan, down_proj)
        out = ops.combine(y, plan, top_k_weights)
        if need_grad:
            # y and act are not kept: the backward recomputes act from gu
            ctx.save_for_backward(hidden_states, top_k_weights, gate_up_proj, down_proj, gu)
            ctx.plan = plan
        return out

    @staticmethod
    def backward(ctx, d_out):
        x, w, gate_up_proj, down_proj, gu = ctx.saved_tensors
        plan = ctx.plan
        need_x, _, need_w, need_w1, need_w2 = ctx.needs_input_grad
        d_out = d_out.to(x.dtype)
        # combine backward fused into GEMM-2's backward (no [S,H] d_y)
        d_gu, act_w, dw = ops.gemm_down_backward_fused(d_out, plan, down_proj, gu, w)
        d_w2 = (ops.gemm_down_backward_dw_gathered(d_out, act_w, plan, down_proj.shape)
                if need_w2 else None)
        del act_w
        d_w1 = (ops.gemm_gate_up_backward_dw(d_gu, x, plan, gate_up_proj.shape)
                if need_w1 else None)
        d_x = None
        if need_x:
            d_xs = ops.gemm_gate_up_backward_dx(d_gu, plan, gate_up_proj)
            d_x = ops.gather_backward(d_xs, plan)
        ctx.plan = None
        return d_x, None, (dw if need_w else None), d_w1, d_w2


def experts_forward(hidden_states: torch.Tensor, top_k_index: torch.Tensor,
                    top_k_weights: torch.Tensor, gate_up_proj: torch.Tensor,
                    down_proj: torch.Tensor) -> torch.Tensor:
    """out[t] = sum_k w[t,k] * down_e(silu(gate_e(x_t)) * up_e(x_t)), e = idx[t,k].

    hidden_states is cast to the weights' dtype (as transformers' _grouped_mm
    does, integrations/moe.py:330-335) and the result is returned in
    hidden_states' dtype (:478)."""
    if hidden_states.dim() != 2:
        raise ValueError("hidden_states must be [T, H]")
    if gate_up_proj.dim() != 3 or down_proj.dim() != 3:
        raise ValueError("gate_up_proj must be [E, 2I, H] and down_proj [E, H, I]")
    E, I2, H = gate_up_proj.shape
    if down_proj.shape != (E, H, I2 // 2) or hidden_states.shape[1] != H:
        raise ValueError(
            f"shape mismatch: hidden {tuple(hidden_states.shape)}, gate_up_proj "
            f"{tuple(gate_up_proj.shape)}, down_proj {tuple(down_proj.shape)}")
    if top_k_index.shape != top_k_weights.shape or top_k_index.shape[0] != hidden_states.shape[0]:
        raise ValueError("top_k_index / top_k_weights must both be [T, K]")
    out_dtype = hidden_states.dtype
    x = hidden_states.to(gate_up_proj.dtype).contiguous()
    out = MoEExpertsFunction.apply(x, top_k_index, top_k_weights.contiguous(),
                                   gate_up_proj.contiguous(), down_proj.contiguous())
    return out.to(out_dtype)


def _check_module(self) -> None:
    if not getattr(self, "has_gate", True):
        raise NotImplementedError("mi355x experts: only gated (gate_up_proj) experts are supported")
    if getattr(self, "has_bias", False):
        raise NotImplementedError("mi355x experts: expert biases are not supported")
    if getattr(self, "is_transposed", False):
        raise NotImplementedError("mi355x experts: transposed expert weights are not supported")
    if not getattr(self, "is_concatenated", True):
        raise NotImplementedError("mi355x experts: interleaved gate/up layout is not supported")
    act = getattr(self, "act_fn", None)
    name = type(act).__name__.lower() if act is not None else "silu"
    if "silu" not in name and "swish" not in name:
        raise NotImplementedError(f"mi355x experts: activation {type(act).__name__} is not SiLU")


def mi355x_experts_forward(self, hidden_states: torch.Tensor, top_k_index: torch.Tensor,
                           top_k_weights: torch.Tensor) -> torch.Tensor:
    """ExpertsInterface entry ("mi355x"), drop-in for grouped_mm_experts_forward
    (transformers/integrations/moe.py:377-478)."""
    _check_module(self)
    return experts_forward(hidden_states, top_k_index, top_k_weights, self.gate_up_proj,
                           self.down_proj)
