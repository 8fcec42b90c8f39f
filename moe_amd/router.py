"""Router modules whose softmax / sigmoid + top-k run in the HIP router kernel.

Both subclass transformers' ``Qwen3MoeTopKRouter`` so that HF's
OutputRecorder keeps capturing index 0 of their output as router_logits
(src/models/modeling_qwen3_moe.py:375-379; the reason the reference's
DeepSeekRouter subclasses it, src/models/router.py:73-79).  By default their
gating linear stays a torch ``F.linear``, so the logits are bit-identical to
the reference's on the same device; ``hip_gating_linear = True`` switches it
to the MFMA kernel (``gating_linear``), whose logits differ only in fp32
summation order (and so can flip a top-k choice between near-tied experts).
"""
from __future__ import annotations

from types import SimpleNamespace

import torch
from torch import nn

from . import library, ops  # noqa: F401  (library registers the moe_amd:: ops)

try:  # the plug-in base class of the reference's routers
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeTopKRouter as _RouterBase
except Exception:  # pragma: no cover - transformers absent: plain module base
    class _RouterBase(nn.Module):  # type: ignore[no-redef]
        def __init__(self, config):
            super().__init__()
            self.top_k = config.num_experts_per_tok
            self.num_experts = config.num_experts
            self.norm_topk_prob = config.norm_topk_prob
            self.hidden_dim = config.hidden_size
            self.weight = nn.Parameter(torch.zeros(self.num_experts, self.hidden_dim))


def router_linear(x: torch.Tensor, weight: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    """logits = x . W^T on the MFMA kernel (bf16 inputs, fp32 accumulation),
    logits in bf16 (F.linear on bf16 tensors, src/models/modeling_qwen3_moe.py:
    268-270) or fp32 (F.linear(h.float(), W.float()), src/models/router.py:
    107-109); differentiable (op ``moe_amd::router_linear``)."""
    return torch.ops.moe_amd.router_linear(x, weight, out_dtype)


def gating_linear(x: torch.Tensor, weight: torch.Tensor, fp32: bool, hip: bool = True):
    """The router's gating linear: bf16 logits (softmax router) or fp32 logits
    (DeepSeek router).  Runs on the MFMA kernel when ``hip`` and both operands
    are bf16 on the GPU (H a multiple of 64, E of 8); otherwise torch's F.linear
    on the same device (the reference's logits bit for bit), whose backward
    runs on the MFMA kernels when the operands are bf16 on the GPU."""
    E, H = weight.shape
    bf = x.is_cuda and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
    if hip and bf and H % 64 == 0 and E % 8 == 0:
        return router_linear(x, weight, torch.float32 if fp32 else torch.bfloat16)
    if bf:
        return torch.ops.moe_amd.torch_gating_linear(x, weight, bool(fp32))
    return ops.torch_gating_linear(x, weight, fp32)


def softmax_topk(logits: torch.Tensor, top_k: int, renormalize: bool = True,
                 logit_offset: torch.Tensor | None = None):
    """(logits) -> (probs fp32 [T,E], weights fp32 [T,K], index [T,K]) with
    the softmax router's backward (op ``moe_amd::softmax_topk``)."""
    return torch.ops.moe_amd.softmax_topk(logits, int(top_k), bool(renormalize), logit_offset)


def sigmoid_topk(logits: torch.Tensor, expert_bias: torch.Tensor | None, top_k: int,
                 renormalize: bool = True, scaling_factor: float | None = None,
                 num_groups: int | None = None, group_topk: int | None = None,
                 weights_dtype: torch.dtype = torch.float32,
                 tokens_per_expert: torch.Tensor | None = None):
    """(fp32 logits) -> (scores, weights, index) for the DeepSeek-V3 router
    (op ``moe_amd::sigmoid_topk``); with ``tokens_per_expert`` the selection
    counts of this call are added to it (src/models/router.py:143-150)."""
    grouped = num_groups is not None and group_topk is not None
    scores, w, idx, counts = torch.ops.moe_amd.sigmoid_topk(
        logits, expert_bias, int(top_k), bool(renormalize), float(scaling_factor or 0.0),
        int(num_groups) if grouped else 0, int(group_topk) if grouped else 0, weights_dtype,
        tokens_per_expert is not None)
    if tokens_per_expert is not None:
        tokens_per_expert.add_(counts)
    return scores, w, idx


def linear_sigmoid_topk(x: torch.Tensor, weight: torch.Tensor, expert_bias: torch.Tensor | None,
                        top_k: int, renormalize: bool = True,
                        scaling_factor: float | None = None, num_groups: int | None = None,
                        group_topk: int | None = None,
                        weights_dtype: torch.dtype = torch.float32,
                        tokens_per_expert: torch.Tensor | None = None):
    """(hidden states) -> (scores, weights, index) of the DeepSeek-V3 router
    with its fp32 gating linear fused into one MFMA kernel (op
    ``moe_amd::linear_sigmoid_topk``); the results of ``gating_linear`` with
    ``hip=True`` followed by ``sigmoid_topk``, bit for bit.  Shapes outside
    the fused kernel's (``ops.router_fused_sigmoid_supported``) take those
    two steps."""
    grouped = num_groups is not None and group_topk is not None
    E = weight.shape[0]
    if not (x.is_cuda and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
            and x.shape[1] % 64 == 0
            and ops.router_fused_sigmoid_supported(E, top_k, num_groups if grouped else None)):
        logits = gating_linear(x, weight, fp32=True, hip=True)
        return sigmoid_topk(logits, expert_bias, top_k, renormalize, scaling_factor, num_groups,
                            group_topk, weights_dtype, tokens_per_expert)
    scores, w, idx, counts = torch.ops.moe_amd.linear_sigmoid_topk(
        x, weight, expert_bias, int(top_k), bool(renormalize), float(scaling_factor or 0.0),
        int(num_groups) if grouped else 0, int(group_topk) if grouped else 0, weights_dtype,
        tokens_per_expert is not None)
    if tokens_per_expert is not None:
        tokens_per_expert.add_(counts)
    return scores, w, idx


class MI355XTopKRouter(_RouterBase):
    """Softmax top-k router (Qwen3MoeTopKRouter.forward,
    src/models/modeling_qwen3_moe.py:266-275): returns
    (router_logits = softmax probs fp32 [T,E], weights fp32 [T,K], index [T,K]).

    ``logit_offset`` (optional [E] fp32 attribute) is added to the logits
    before the softmax; the skewed-routing benchmark config uses it."""

    hip_gating_linear = False  # True: MFMA gating linear (see module docstring)

    def __init__(self, config):
        super().__init__(config)
        self.logit_offset: torch.Tensor | None = None

    def forward(self, hidden_states):
        hidden_states = hidden_states.reshape(-1, self.hidden_dim)
        logits = gating_linear(hidden_states, self.weight, fp32=False, hip=self.hip_gating_linear)
        return softmax_topk(logits, self.top_k, bool(self.norm_topk_prob), self.logit_offset)

    @classmethod
    def from_router(cls, old: nn.Module) -> "MI355XTopKRouter":
        cfg = SimpleNamespace(num_experts_per_tok=old.top_k, num_experts=old.num_experts,
                              norm_topk_prob=old.norm_topk_prob, hidden_size=old.hidden_dim)
        new = cls(cfg)
        new.weight = old.weight  # share the Parameter: optimizer state and ckpt keys unchanged
        new.logit_offset = getattr(old, "logit_offset", None)
        return new


class MI355XDeepSeekRouter(_RouterBase):
    """DeepSeek-V3 sigmoid + expert-bias router (src/models/router.py:73-155):
    fp32 gating linear, sigmoid scores, biased (optionally group-limited)
    top-k, unbiased renormalised weights (+1e-20) times topk_scaling_factor,
    cast to the hidden dtype.  Keeps the reference's buffers:
    ``expert_bias`` (persistent), ``local_tokens_per_expert`` (non-persistent,
    incremented only when grad is enabled) and ``_last_top_k_idx``."""

    def __init__(self, config):
        super().__init__(config)
        self.scaling_factor = getattr(config, "topk_scaling_factor", None)
        self.num_groups = getattr(config, "num_groups", None)
        self.group_topk = getattr(config, "group_topk", None)
        self.register_buffer("expert_bias", torch.zeros(self.num_experts, dtype=torch.float32))
        self.register_buffer("local_tokens_per_expert",
                             torch.zeros(self.num_experts, dtype=torch.float32), persistent=False)
        self._last_top_k_idx = None

    hip_gating_linear = False  # True: MFMA gating linear with fp32 logits
    fused_router = False       # True: that gating linear with the router in its epilogue

    def forward(self, hidden_states):
        hidden_states = hidden_states.reshape(-1, self.hidden_dim)
        counting = torch.is_grad_enabled()
        tpe = self.local_tokens_per_expert if counting else None
        if self.fused_router:
            scores, w, idx = linear_sigmoid_topk(
                hidden_states, self.weight, self.expert_bias, self.top_k,
                bool(self.norm_topk_prob), self.scaling_factor, self.num_groups, self.group_topk,
                hidden_states.dtype, tpe)
            self._last_top_k_idx = idx.detach()
            return scores, w, idx
        logits = gating_linear(hidden_states, self.weight, fp32=True, hip=self.hip_gating_linear)
        scores, w, idx = sigmoid_topk(
            logits, self.expert_bias, self.top_k, bool(self.norm_topk_prob), self.scaling_factor,
            self.num_groups, self.group_topk, hidden_states.dtype, tpe)
        self._last_top_k_idx = idx.detach()
        return scores, w, idx

    @classmethod
    def from_router(cls, old: nn.Module) -> "MI355XDeepSeekRouter":
        cfg = SimpleNamespace(num_experts_per_tok=old.top_k, num_experts=old.num_experts,
                              norm_topk_prob=old.norm_topk_prob, hidden_size=old.hidden_dim,
                              topk_scaling_factor=getattr(old, "scaling_factor", None),
                              num_groups=getattr(old, "num_groups", None),
                              group_topk=getattr(old, "group_topk", None))
        new = cls(cfg)
        new.weight = old.weight
        new.expert_bias = old.expert_bias
        new.local_tokens_per_expert = old.local_tokens_per_expert
        new._last_top_k_idx = getattr(old, "_last_top_k_idx", None)
        return new
