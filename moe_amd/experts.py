"""The expert layer: permute -> grouped GEMM-1 + SwiGLU -> grouped GEMM-2 ->
combine, with a hand-written backward, all on the HIP kernels.

``experts_forward`` is the functional form, a call of the differentiable
custom op ``moe_amd::experts_fwd`` (fake and autograd registered, so
torch.compile traces it without a graph break, as the reference's backend
registers its grouped GEMM, integrations/moe.py:245-257; backward op
``moe_amd::experts_bwd``, formulas :226-242, the combine's backward fused
into GEMM-2's).  ``mi355x_experts_forward`` has the transformers
ExpertsInterface signature
``fn(self, hidden_states [T,H], top_k_index [T,K], top_k_weights [T,K])``
(transformers/integrations/moe.py:377-382) and reads the bank's
``gate_up_proj [E,2I,H]`` / ``down_proj [E,H,I]`` from ``self``.
"""
from __future__ import annotations

import torch

from . import library  # noqa: F401  (registers the moe_amd:: ops)


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
    w = top_k_weights.contiguous()
    save = torch.is_grad_enabled() and any(t.requires_grad
                                           for t in (x, w, gate_up_proj, down_proj))
    out = torch.ops.moe_amd.experts_fwd(x, top_k_index, w, gate_up_proj.contiguous(),
                                        down_proj.contiguous(), save)[0]
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
