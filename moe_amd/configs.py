"""The benchmark workloads (the five expert-layer shapes the reference's
configs/scaling/*.yaml define) and their seeded synthetic inputs.

Inputs are drawn in fp32 on the CPU from ``torch.Generator().manual_seed(seed)``
in a fixed order -- x, W_router, gate_up_proj [E,2I,H], down_proj [E,H,I],
the config extra (logit offset or expert bias), dout -- then cast to the
config dtype, so a CPU and a GPU run see identical bits.  Weights ~ N(0, 0.02)
as the reference initialises them (src/models/modeling_qwen3_moe.py:381-389);
x, dout ~ N(0, 1).
"""
from __future__ import annotations

from dataclasses import dataclass, replace

import torch


@dataclass(frozen=True)
class LayerConfig:
    name: str
    T: int
    H: int
    E: int
    K: int
    I: int
    dtype: torch.dtype
    router: str = "softmax"        # "softmax" | "sigmoid"
    skew: float = 0.0              # Zipf logit offset scale (M config)
    zipf_s: float = 1.1
    bias_range: float = 0.0        # DeepSeek expert_bias ~ U(-r, r)
    backward: bool = True
    # layer calls whose weight gradients sum into one bank gradient per
    # optimizer step: the layers sharing a global bank x gradient-accumulation
    # micro-batches (configs/scaling/xs_global.yaml: 16 layers, 1;
    # retrofit_1.7b_global.yaml: 28 layers, 2); 1 for a per-layer bank
    bank_calls: int = 1

    @property
    def S(self) -> int:
        return self.T * self.K

    def gemm_flops(self, backward: bool | None = None) -> float:
        """Algorithmic grouped-GEMM FLOPs: 6*S*H*I forward, 18*S*H*I fwd+bwd."""
        bw = self.backward if backward is None else backward
        return (18.0 if bw else 6.0) * self.S * self.H * self.I

    def scaled(self, T: int) -> "LayerConfig":
        return replace(self, T=T)


CONFIGS: dict[str, LayerConfig] = {
    "xs_std": LayerConfig("XS standard", 2048, 1024, 16, 4, 768, torch.float32, backward=False),
    "xs_global": LayerConfig("XS global shared bank", 16384, 1024, 128, 4, 768, torch.bfloat16,
                             bank_calls=16),
    "m_skew": LayerConfig("M standard, Zipf-skewed", 32768, 2048, 128, 8, 768, torch.bfloat16,
                          skew=2.0),
    "l": LayerConfig("L (Qwen3-30B-A3B)", 65536, 2048, 128, 8, 768, torch.bfloat16),
    "retrofit": LayerConfig("Retrofit 1.7B global bank", 16384, 2048, 1792, 8, 768,
                            torch.bfloat16, router="sigmoid", bias_range=0.5, bank_calls=56),
}


@dataclass
class LayerInputs:
    x: torch.Tensor
    w_router: torch.Tensor
    gate_up_proj: torch.Tensor
    down_proj: torch.Tensor
    logit_offset: torch.Tensor | None
    expert_bias: torch.Tensor | None
    dout: torch.Tensor


def make_inputs(cfg: LayerConfig, seed: int = 0, device: str | torch.device = "cpu"
                ) -> LayerInputs:
    """Seeded inputs in the fixed draw order, cast to cfg.dtype on `device`.

    Every tensor is drawn on the CPU; the expert banks one expert at a time
    (each expert's fp32 draw is cast and copied to `device` before the next
    is drawn), so even the 1792-expert bank needs no multi-GB host buffer
    and a CPU and a GPU run see identical bits."""
    g = torch.Generator().manual_seed(seed)
    dt = cfg.dtype
    x = torch.randn(cfg.T, cfg.H, generator=g).to(dt).to(device)
    w_router = (torch.randn(cfg.E, cfg.H, generator=g) * 0.02).to(dt).to(device)
    w1 = torch.empty(cfg.E, 2 * cfg.I, cfg.H, dtype=dt, device=device)
    w2 = torch.empty(cfg.E, cfg.H, cfg.I, dtype=dt, device=device)
    for e in range(cfg.E):
        w1[e] = (torch.randn(2 * cfg.I, cfg.H, generator=g) * 0.02).to(dt)
    for e in range(cfg.E):
        w2[e] = (torch.randn(cfg.H, cfg.I, generator=g) * 0.02).to(dt)
    offset = bias = None
    if cfg.skew:
        rank = torch.randperm(cfg.E, generator=g).to(torch.float32) + 1.0
        offset = (cfg.skew * rank.pow(-cfg.zipf_s)).to(device)
    if cfg.bias_range:
        bias = ((torch.rand(cfg.E, generator=g) * 2.0 - 1.0) * cfg.bias_range).to(device)
    dout = torch.randn(cfg.T, cfg.H, generator=g).to(dt).to(device)
    return LayerInputs(x, w_router, w1, w2, offset, bias, dout)
