"""transformers integration: the "mi355x" ExpertsInterface key and install().

``register()`` adds ``"mi355x"`` to transformers' ExpertsInterface
(transformers/integrations/moe.py:481-506; class-wide registry of
utils/generic.py GeneralInterface).  ``install(model)`` then swaps every
Qwen3MoeTopKRouter-derived gate for its HIP counterpart in place (as
src/models/standard_moe.py:72-78 swaps in DeepSeekRouter) and selects the
experts implementation with ``model.set_experts_implementation("mi355x")``
(the call train.py:239-245 makes with "grouped_mm").  Both the per-layer
banks (Qwen3MoeSparseMoeBlock.experts) and the global shared bank
(GlobalMoEModel.global_experts) dispatch through that key unchanged.
"""
from __future__ import annotations

from torch import nn

from .experts import mi355x_experts_forward
from .router import MI355XDeepSeekRouter, MI355XTopKRouter, _RouterBase

EXPERTS_KEY = "mi355x"


def register() -> None:
    from transformers.integrations.moe import ExpertsInterface
    ExpertsInterface.register(EXPERTS_KEY, mi355x_experts_forward)


def swap_routers(model: nn.Module) -> int:
    """Replaces each router (a Qwen3MoeTopKRouter or subclass) by the HIP one.
    Routers carrying an ``expert_bias`` buffer become MI355XDeepSeekRouter.
    Parameters and buffers are shared, so state_dict keys are unchanged.
    Returns the number of routers swapped."""
    n = 0
    for parent in list(model.modules()):
        for name, child in list(parent.named_children()):
            if isinstance(child, (MI355XTopKRouter, MI355XDeepSeekRouter)):
                continue
            if not isinstance(child, _RouterBase):
                continue
            cls = MI355XDeepSeekRouter if hasattr(child, "expert_bias") else MI355XTopKRouter
            new = cls.from_router(child)
            new.train(child.training)
            setattr(parent, name, new)
            n += 1
    return n


def install(model: nn.Module, routers: bool = True, experts: bool = True) -> nn.Module:
    register()
    if routers:
        swap_routers(model)
    if experts:
        model.set_experts_implementation(EXPERTS_KEY)
    return model
