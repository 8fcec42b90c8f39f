"""CPU oracle for the routing consumers — TEST INFRASTRUCTURE ONLY.

Restates, in fp64 torch on the CPU, the functions that consume the router's
outputs right after the MoE layer: the two load-balancing losses, the routing
statistics and the aux-loss-free expert-bias update.  Only ``tests/`` use it,
as the checker; the product package ``moe_amd`` never imports it.

Reference (leonmodal/moe):
  load_balancing_loss_func      src/models/load_balancing.py:19-90
  seq_load_balancing_loss_func  src/models/load_balancing.py:93-169
  accumulate_expert_counts      src/utils/routing_stats.py:53-80
  compute_routing_stats         src/utils/routing_stats.py:113-220
  update_expert_biases          train.py:79-139

Top-k ties: the reference calls torch.topk, whose order among exactly equal
values is implementation-defined (on ROCm it is not by index); this oracle
and the kernels keep the lower expert id first.  Every quantity below that
depends on the selection is therefore compared on inputs without exact ties,
or through closed forms that do not depend on which tied expert is picked.

How each function is pinned (tests/test_oracle_balancing.py):
  switch_aux_loss      the reference tests' closed forms (uniform probs give
                       top_k; tests/test_aux_loss_fix.py:9-14) and skew bounds;
                       a per-token one-hot loop with explicit attention-mask
                       weights; gradient by finite differences
  seq_aux_loss         the DeepSeek-V3 paper (Eqs. 17-20) and Megatron-LM forms
                       restated from tests/test_seq_loss_vs_paper.py:24-101
                       (an independent per-sequence loop); 1.0 at balanced
                       routing; gradient by finite differences
  routing_stats        closed forms: uniform (imbalance 1, cv 0, entropy 1),
                       collapsed (imbalance E, entropy 0), identical and
                       disjoint layers (cross-layer similarity 1 and 0);
                       margins from a full sort
  update_expert_biases Megatron-LM's get_updated_expert_bias (restated from
                       tests/test_bias_update_detailed.py:97-102) per layer;
                       the global and blended forms by hand-derived cases
"""
from __future__ import annotations

import math

import torch

from .moe_oracle import rank_topk


def _counts(probs: torch.Tensor, top_k: int, weights: torch.Tensor | None = None):
    """Per-expert number of top-k selections (optionally token-weighted)."""
    T, E = probs.shape
    _, idx = rank_topk(probs, top_k)
    w = torch.ones(T, dtype=torch.float64) if weights is None else weights.double()
    c = torch.zeros(E, dtype=torch.float64)
    c.index_add_(0, idx.reshape(-1), w.repeat_interleave(top_k))
    return c


def switch_aux_loss(gate_logits, num_experts: int, top_k: int = 2,
                    attention_mask: torch.Tensor | None = None) -> torch.Tensor:
    """load_balancing.py:19-90 (Switch Transformer loss on router
    probabilities, no second softmax, f_i kept local).  Layers are
    concatenated along tokens; with an attention mask [B, S] each token's
    selections and probabilities are weighted by its mask value.  Returns an
    fp64 scalar, differentiable in every layer's probs."""
    probs = torch.cat([g.double() for g in gate_logits], dim=0)
    n_layers = len(gate_logits)
    if attention_mask is None:
        w = torch.ones(probs.shape[0], dtype=torch.float64)
    else:
        w = attention_mask.double().reshape(-1).repeat(n_layers)
    denom = w.sum()
    tokens_per_expert = _counts(probs.detach(), top_k, w) / denom        # sum over k of [K, E]
    router_prob_per_expert = (probs * w[:, None]).sum(dim=0) / denom
    return (tokens_per_expert * router_prob_per_expert).sum() * num_experts


def seq_aux_loss(gate_logits, num_experts: int, top_k: int = 2, batch_size: int = 1,
                 selected_experts=None) -> torch.Tensor:
    """load_balancing.py:93-169 (DeepSeek-V3 sequence-wise loss, Eqs. 17-20):
    per layer and sequence, scores normalised per token (eps 1e-20), f_i =
    E / (K * S) * selections of expert i in the sequence (the given routed
    indices, or top-k of the normalised scores), P_i = mean normalised score;
    loss = mean over sequences of sum_i f_i P_i, averaged over layers."""
    total = torch.zeros((), dtype=torch.float64)
    for li, g in enumerate(gate_logits):
        T, E = g.shape
        S = T // batch_size
        s = g.double()
        s = s / (s.sum(dim=-1, keepdim=True) + 1e-20)
        sel = None
        if selected_experts is not None and li < len(selected_experts):
            cand = selected_experts[li]
            if cand is not None and tuple(cand.shape) == (T, top_k):
                sel = cand.reshape(-1).to(torch.int64)
        if sel is None:
            _, sel = rank_topk(s.detach(), top_k)
            sel = sel.reshape(-1)
        counts = torch.zeros(batch_size, num_experts, dtype=torch.float64)
        seq = torch.arange(T).repeat_interleave(top_k) // S
        counts.index_put_((seq, sel), torch.ones(T * top_k, dtype=torch.float64),
                          accumulate=True)
        f = counts * (num_experts / (top_k * S))
        P = s.reshape(batch_size, S, E).mean(dim=1)
        total = total + (f * P).sum(dim=-1).mean()
    return total / len(gate_logits)


def routing_stats(router_logits, num_experts_per_tok: int, is_global: bool = False) -> dict:
    """routing_stats.py:113-220, with its keys and definitions (torch.std is
    the unbiased estimate; argmax takes the first maximum)."""
    K = num_experts_per_tok
    stats: dict = {}
    loads = []
    for li, probs in enumerate(router_logits):
        p = probs.detach().double()
        T, E = p.shape
        tag = f"routing/layer_{li:02d}"
        counts = _counts(p, K)
        total = float(T * K)
        ideal = total / E
        stats[f"{tag}_load_imbalance"] = float(counts.max() / ideal)
        stats[f"{tag}_load_cv"] = float(counts.std() / counts.mean()) if counts.mean() > 0 else 0.0
        stats[f"{tag}_num_active_experts"] = int((counts > 0).sum())
        stats[f"{tag}_top_expert"] = int(counts.argmax())
        stats[f"_hist/{tag}_expert_load_frac"] = (counts / total).tolist()
        dist = counts / (counts.sum() + 1e-10)
        ent = float(-(dist * (dist + 1e-10).log()).sum())
        stats[f"{tag}_entropy"] = ent / math.log(E) if E > 1 else 0.0
        if E > K:
            srt = p.sort(dim=-1, descending=True).values
            margin = srt[:, K - 1] - srt[:, K]
            stats[f"{tag}_router_margin_mean"] = float(margin.mean())
            stats[f"{tag}_router_margin_min"] = float(margin.min())
        loads.append(counts)
    if is_global and len(loads) > 1:
        mat = torch.stack(loads)
        normed = mat / mat.norm(dim=1, keepdim=True).clamp(min=1e-10)
        sim = normed @ normed.T
        L = sim.shape[0]
        off = sim[torch.triu(torch.ones(L, L, dtype=torch.bool), diagonal=1)]
        stats["routing/cross_layer_sim_mean"] = float(off.mean())
        stats["routing/cross_layer_sim_min"] = float(off.min())
        stats["routing/cross_layer_sim_max"] = float(off.max())
        E = mat.shape[1]
        stats["_hist/global_expert_layer_count"] = (mat > 0).double().sum(dim=0).tolist()
        pool = mat.sum(dim=0)
        ptot = float(pool.sum())
        stats["routing/global_pool_load_imbalance"] = float(pool.max() / (ptot / E))
        stats["routing/global_pool_load_cv"] = float(pool.std() / pool.mean()) if pool.mean() > 0 else 0.0
        stats["routing/global_pool_num_active"] = int((pool > 0).sum())
        stats["routing/global_pool_top_expert"] = int(pool.argmax())
        frac = pool / ptot
        stats["_hist/global_pool_expert_load_frac"] = frac.tolist()
        pent = float(-(frac * (frac + 1e-10).log()).sum())
        stats["routing/global_pool_entropy"] = pent / math.log(E) if E > 1 else 0.0
    return stats


def update_expert_biases(counts, biases, update_rate: float, is_global: bool = False,
                         alpha: float = 0.0):
    """train.py:79-139 without the DDP all-reduce: per-layer (or pooled, or
    alpha-blended) sign(mean - counts) * rate added to each bias, in the
    buffers' fp32 with the reference's operation order (counts are integers,
    so every sum and mean is exact up to its final rounding).  Returns
    (new biases, stats dict)."""
    counts = [c.float() for c in counts]
    new = [b.float().clone() for b in biases]
    if is_global:
        pool = torch.stack(counts).sum(dim=0)
        gdelta = torch.sign(pool.mean() - pool) * update_rate
        for i, c in enumerate(counts):
            if alpha > 0:
                ldelta = torch.sign(c.mean() - c) * update_rate
                new[i] += alpha * ldelta + (1 - alpha) * gdelta
            else:
                new[i] += gdelta
    else:
        for i, c in enumerate(counts):
            new[i] += torch.sign(c.mean() - c) * update_rate
    allb = torch.cat(new).double()
    stats = {"routing/expert_bias_mean": float(allb.mean()),
             "routing/expert_bias_std": float(allb.std()),
             "routing/expert_bias_min": float(allb.min()),
             "routing/expert_bias_max": float(allb.max())}
    return new, stats
