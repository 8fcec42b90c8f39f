"""moe_amd — MI355X (gfx950) HIP implementation of the Qwen3-MoE expert layer.

Public API:
  experts_forward(hidden_states, top_k_index, top_k_weights, gate_up_proj, down_proj)
  mi355x_experts_forward(self, hidden_states, top_k_index, top_k_weights)   # ExpertsInterface
  MI355XTopKRouter / MI355XDeepSeekRouter                                     # router modules
  hf.register() / hf.install(model)                                           # transformers hook
  ops.*                                                                       # one wrapper per C entry
  torch.ops.moe_amd.*                                                         # custom ops (library.py)
"""
from . import library, ops
from .experts import experts_forward, mi355x_experts_forward
from .router import MI355XDeepSeekRouter, MI355XTopKRouter

__all__ = [
    "ops",
    "library",
    "experts_forward",
    "mi355x_experts_forward",
    "MI355XTopKRouter",
    "MI355XDeepSeekRouter",
]
