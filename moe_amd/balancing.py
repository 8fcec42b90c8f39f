"""Routing consumers on the GPU: the load-balancing losses, the routing
statistics and the aux-loss-free expert-bias update, as drop-in replacements
for the reference functions of the same names and arguments:

  load_balancing_loss_func       src/models/load_balancing.py:19-90
  seq_load_balancing_loss_func   src/models/load_balancing.py:93-169
  accumulate_expert_counts       src/utils/routing_stats.py:53-80
  expert_counts_to_tables        src/utils/routing_stats.py:83-110
  compute_routing_stats          src/utils/routing_stats.py:113-220
  update_expert_biases           train.py:79-139

The [T, E] passes (top-k selection counts, probability column sums, margins,
sequence statistics, both loss gradients, the bias update) are HIP kernels
(``moe_amd_topk_stats`` and friends); the O(E) assembly of the scalars runs
on the same device, and ``compute_routing_stats`` reads all of its values
back with one transfer where the reference reads each with ``.item()``.

Differences from the reference, all at ties or rounding level: the top-k
keeps the lower expert id among exactly equal values (torch.topk's order is
implementation-defined); sums accumulate in fp64 in a fixed order.
"""
from __future__ import annotations

import math
from typing import Sequence

import torch

from . import _lib
from .ops import _call, _dtype_code, _need_cuda, _stream, on_tensor_device


def _contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _as_probs(t: torch.Tensor) -> torch.Tensor:
    if t.dtype not in (torch.float32, torch.bfloat16):
        t = t.float()
    return _contig(t)


@on_tensor_device
def topk_stats(probs: torch.Tensor, top_k: int, token_weights: torch.Tensor | None = None):
    """(counts [E] fp64, prob_sums [E] fp64, margin [2] fp64 = sum and min of
    the k-th minus (k+1)-th largest value) of one layer's [T, E] values."""
    _need_cuda(probs, token_weights)
    probs = _as_probs(probs)
    T, E = probs.shape
    dev = probs.device
    w = None
    if token_weights is not None:
        w = _contig(token_weights.reshape(-1).to(device=dev, dtype=torch.float32))
        if w.numel() != T:
            raise ValueError(f"token weights: {w.numel()} values for {T} tokens")
    nbytes = int(_lib.load().moe_amd_topk_stats_workspace_size(T, E))
    ws = torch.empty(max(nbytes, 16), device=dev, dtype=torch.uint8)
    out = torch.empty(2 * E + 2, device=dev, dtype=torch.float64)
    _call("moe_amd_topk_stats", probs.data_ptr() if T else None, _dtype_code(probs.dtype),
          w.data_ptr() if w is not None else None, T, E, top_k, ws.data_ptr(), ws.numel(),
          out.data_ptr(), out[E:].data_ptr(), out[2 * E:].data_ptr(), _stream(probs))
    return out[:E], out[E:2 * E], out[2 * E:]


# ---------------------------------------------------------- Switch loss

class SwitchAuxLoss(torch.autograd.Function):
    """E * sum_e f_e * p_e over the concatenated layers (load_balancing.py:
    40-90): f_e the (mask-weighted) fraction of tokens whose top-k holds e,
    p_e the (mask-weighted) mean probability.  Gradient w.r.t. layer l's
    probs: E * f_e / denom * w_t, f non-differentiable (hard assignment)."""

    @staticmethod
    def forward(ctx, num_experts, top_k, token_weights, *layers):
        counts = sums = None
        for g in layers:
            c, s, _ = topk_stats(g, top_k, token_weights)
            counts = c if counts is None else counts + c
            sums = s if sums is None else sums + s
        # the number of (mask-weighted) tokens over all layers
        if token_weights is not None:
            denom_t = token_weights.to(torch.float64).sum() * len(layers)
        else:
            denom_t = torch.tensor(float(sum(g.shape[0] for g in layers)), dtype=torch.float64,
                                   device=counts.device)
        tpe = counts / denom_t
        loss = (tpe * (sums / denom_t)).sum() * num_experts
        ctx.coef = tpe * (num_experts / denom_t)
        ctx.token_weights = token_weights
        ctx.meta = [(g.shape, g.dtype) for g in layers]
        return loss.to(layers[0].dtype if layers[0].is_floating_point() else torch.float32)

    @staticmethod
    @on_tensor_device
    def backward(ctx, g):
        coef = _contig(ctx.coef * g.to(torch.float64))
        w = ctx.token_weights
        grads = []
        for shape, dt in ctx.meta:
            T, E = shape
            gdt = dt if dt in (torch.float32, torch.bfloat16) else torch.float32
            out = torch.empty(T, E, device=coef.device, dtype=gdt)
            _call("moe_amd_switch_aux_backward", coef.data_ptr(),
                  w.data_ptr() if w is not None else None, T, E, _dtype_code(gdt),
                  out.data_ptr(), _stream(coef))
            grads.append(out.to(dt))
        return (None, None, None, *grads)


def load_balancing_loss_func(gate_logits, num_experts: int | None = None, top_k: int = 2,
                             attention_mask: torch.Tensor | None = None):
    """Switch-Transformer load-balancing loss on router probabilities
    (src/models/load_balancing.py:19-90): ``gate_logits`` is the tuple of
    per-layer [T, E] softmax probabilities; returns 0 when it is None or not a
    tuple, like the reference."""
    if gate_logits is None or not isinstance(gate_logits, tuple):
        return 0
    dev = gate_logits[0].device
    layers = [g.to(dev) for g in gate_logits]
    E = num_experts if num_experts is not None else layers[0].shape[-1]
    w = None
    if attention_mask is not None:
        w = _contig(attention_mask.to(device=dev, dtype=torch.float32).reshape(-1))
        if layers[0].shape[0] != w.numel():
            raise ValueError("attention_mask must hold one value per token of a layer")
    return SwitchAuxLoss.apply(E, top_k, w, *layers)


# ------------------------------------------------ sequence-wise (DeepSeek)

class SeqAuxLoss(torch.autograd.Function):
    """Mean over layers and sequences of sum_e f_e P_e (load_balancing.py:
    93-169): P the mean over the sequence of the per-token normalised scores,
    f = E / (K S) * selections.  Gradient through P and the normalisation."""

    @staticmethod
    @on_tensor_device
    def forward(ctx, num_experts, top_k, batch_size, selected, *layers):
        total = None
        ctx.saved = []
        L = len(layers)
        for li, g in enumerate(layers):
            _need_cuda(g)
            s = _as_probs(g)
            T, E = s.shape
            S = T // batch_size
            sel = None
            if selected is not None and li < len(selected):
                cand = selected[li]
                if cand is not None and tuple(cand.shape) == (T, top_k):
                    sel = _contig(cand.to(device=s.device, dtype=torch.int64))
            nbytes = int(_lib.load().moe_amd_seq_stats_workspace_size(T, E, batch_size))
            if nbytes == 0:
                raise ValueError(f"seq load-balancing loss: {T} tokens do not split into "
                                 f"{batch_size} sequences")
            ws = torch.empty(nbytes, device=s.device, dtype=torch.uint8)
            cnt = torch.empty(batch_size, E, device=s.device, dtype=torch.float64)
            P = torch.empty_like(cnt)
            _call("moe_amd_seq_stats", s.data_ptr(), _dtype_code(s.dtype),
                  sel.data_ptr() if sel is not None else None, T, E, top_k, batch_size,
                  ws.data_ptr(), ws.numel(), cnt.data_ptr(), P.data_ptr(), _stream(s))
            f = cnt * (num_experts / (top_k * S))
            layer_loss = (f * P).sum(dim=-1).mean()
            total = layer_loss if total is None else total + layer_loss
            ctx.saved.append((s, f / (L * batch_size * S), g.dtype))
        ctx.batch_size = batch_size
        return (total / L).to(torch.float32)

    @staticmethod
    @on_tensor_device
    def backward(ctx, g):
        grads = []
        for s, coef, dt in ctx.saved:
            T, E = s.shape
            c = _contig(coef * g.to(torch.float64))
            out = torch.empty(T, E, device=s.device, dtype=s.dtype)
            _call("moe_amd_seq_aux_backward", s.data_ptr(), _dtype_code(s.dtype), c.data_ptr(),
                  T, E, ctx.batch_size, out.data_ptr(), _stream(s))
            grads.append(out.to(dt))
        ctx.saved = None
        return (None, None, None, None, *grads)


def seq_load_balancing_loss_func(gate_logits, num_experts: int | None = None, top_k: int = 2,
                                 batch_size: int = 1, selected_experts=None):
    """DeepSeek-V3 sequence-wise load-balancing loss (Eqs. 17-20,
    src/models/load_balancing.py:93-169); ``selected_experts`` are the routed
    indices per layer ([T, K]) when available.  Returns 0 for a None or
    non-tuple input, like the reference."""
    if gate_logits is None or not isinstance(gate_logits, tuple):
        return 0
    E = num_experts if num_experts is not None else gate_logits[0].shape[-1]
    return SeqAuxLoss.apply(E, top_k, batch_size, selected_experts, *gate_logits)


# ----------------------------------------------------------- statistics

def accumulate_expert_counts(router_logits: Sequence[torch.Tensor], num_experts_per_tok: int,
                             accumulator: dict | None = None) -> dict:
    """Adds each layer's per-expert selection counts (float32 [E], on the
    device) to ``accumulator`` (routing_stats.py:53-80)."""
    if accumulator is None:
        accumulator = {}
    for li, probs in enumerate(router_logits):
        counts, _, _ = topk_stats(probs.detach(), num_experts_per_tok)
        c = counts.to(torch.float32)
        if li in accumulator:
            accumulator[li] += c
        else:
            accumulator[li] = c
    return accumulator


def expert_counts_to_tables(accumulator: dict, is_global: bool = False) -> dict:
    """``_table/`` entries of accumulated counts (routing_stats.py:83-110)."""
    stats = {}
    for li in sorted(accumulator):
        counts = accumulator[li]
        tag = f"routing/layer_{li:02d}"
        stats[f"_table/{tag}_expert_tokens"] = list(zip(range(counts.shape[0]),
                                                        counts.cpu().tolist()))
    if is_global and len(accumulator) > 1:
        pool = torch.stack([accumulator[i] for i in sorted(accumulator)]).sum(dim=0)
        stats["_table/global_pool_expert_tokens"] = list(zip(range(pool.shape[0]),
                                                             pool.cpu().tolist()))
    return stats


def _entropy(frac: torch.Tensor) -> torch.Tensor:
    return -(frac * (frac + 1e-10).log()).sum()


def compute_routing_stats(router_logits: Sequence[torch.Tensor], num_experts_per_tok: int,
                          is_global: bool = False) -> dict:
    """Per-layer load imbalance, CV, active experts, top expert, load
    fractions, entropy and router margins, plus the cross-layer and pooled
    metrics for a global bank (routing_stats.py:113-220, same keys)."""
    K = num_experts_per_tok
    scalars: list[tuple[str, torch.Tensor, type]] = []
    hists: list[tuple[str, torch.Tensor]] = []
    loads = []
    for li, probs in enumerate(router_logits):
        T, E = probs.shape
        tag = f"routing/layer_{li:02d}"
        counts, _, margin = topk_stats(probs.detach(), K)
        total = float(T * K)
        mean = counts.mean()
        scalars.append((f"{tag}_load_imbalance", counts.max() / (total / E), float))
        scalars.append((f"{tag}_load_cv", torch.where(mean > 0, counts.std() / mean,
                                                       torch.zeros_like(mean)), float))
        scalars.append((f"{tag}_num_active_experts", (counts > 0).sum(), int))
        scalars.append((f"{tag}_top_expert", counts.argmax(), int))
        hists.append((f"_hist/{tag}_expert_load_frac", counts / total))
        dist = counts / (counts.sum() + 1e-10)
        scalars.append((f"{tag}_entropy", _entropy(dist) / math.log(E) if E > 1
                        else torch.zeros_like(mean), float))
        if E > K:
            scalars.append((f"{tag}_router_margin_mean", margin[0] / T, float))
            scalars.append((f"{tag}_router_margin_min", margin[1], float))
        loads.append(counts)
    if is_global and len(loads) > 1:
        mat = torch.stack(loads)
        normed = mat / mat.norm(dim=1, keepdim=True).clamp(min=1e-10)
        sim = normed @ normed.T
        L = sim.shape[0]
        off = sim[torch.triu(torch.ones(L, L, dtype=torch.bool, device=sim.device), diagonal=1)]
        scalars.append(("routing/cross_layer_sim_mean", off.mean(), float))
        scalars.append(("routing/cross_layer_sim_min", off.min(), float))
        scalars.append(("routing/cross_layer_sim_max", off.max(), float))
        E = mat.shape[1]
        hists.append(("_hist/global_expert_layer_count", (mat > 0).to(torch.float64).sum(dim=0)))
        pool = mat.sum(dim=0)
        ptot = pool.sum()
        pmean = pool.mean()
        scalars.append(("routing/global_pool_load_imbalance", pool.max() / (ptot / E), float))
        scalars.append(("routing/global_pool_load_cv", torch.where(
            pmean > 0, pool.std() / pmean, torch.zeros_like(pmean)), float))
        scalars.append(("routing/global_pool_num_active", (pool > 0).sum(), int))
        scalars.append(("routing/global_pool_top_expert", pool.argmax(), int))
        frac = pool / ptot
        hists.append(("_hist/global_pool_expert_load_frac", frac))
        scalars.append(("routing/global_pool_entropy", _entropy(frac) / math.log(E) if E > 1
                        else torch.zeros_like(pmean), float))
    # one device-to-host transfer for every value
    flat = torch.cat([v.reshape(1).to(torch.float64) for _, v, _ in scalars] +
                     [h.reshape(-1).to(torch.float64) for _, h in hists]).cpu().tolist()
    stats: dict = {}
    i = 0
    for name, _, kind in scalars:
        stats[name] = kind(flat[i]) if kind is int else flat[i]
        i += 1
    for name, h in hists:
        stats[name] = flat[i:i + h.numel()]
        i += h.numel()
    return stats


# ---------------------------------------------------- expert-bias update

def _bias_routers(model) -> list:
    return [m for m in model.modules()
            if isinstance(getattr(m, "expert_bias", None), torch.Tensor)
            and isinstance(getattr(m, "local_tokens_per_expert", None), torch.Tensor)]


def update_expert_biases(model, update_rate: float, accelerator=None, is_global: bool = False,
                         alpha: float = 0.0) -> dict:
    """Aux-loss-free balancing step (train.py:79-139): every router carrying
    ``expert_bias`` and ``local_tokens_per_expert`` (the reference's
    DeepSeekRouter and MI355XDeepSeekRouter) moves its bias by
    sign(mean - count) * rate (per layer, pooled, or alpha-blended) in one
    kernel launch; the counts are zeroed.  With several processes the counts
    are all-reduced first, as in the reference.  Returns the bias stats."""
    routers = _bias_routers(model)
    if not routers:
        return {}
    counts = [r.local_tokens_per_expert for r in routers]
    biases = [r.expert_bias for r in routers]
    _need_cuda(*counts, *biases)
    E = biases[0].numel()
    for c, b in zip(counts, biases):
        if (c.dtype != torch.float32 or b.dtype != torch.float32 or c.numel() != E
                or b.numel() != E or not c.is_contiguous() or not b.is_contiguous()):
            raise RuntimeError("update_expert_biases: routers need contiguous fp32 [E] buffers")
    if accelerator is not None and getattr(accelerator, "num_processes", 1) > 1:
        for c in counts:
            torch.distributed.all_reduce(c, op=torch.distributed.ReduceOp.SUM)
    dev = biases[0].device
    ptrs = torch.tensor([c.data_ptr() for c in counts] + [b.data_ptr() for b in biases],
                        dtype=torch.int64, device=dev)
    stats = torch.empty(4, dtype=torch.float64, device=dev)
    L = len(routers)
    with torch.cuda.device(dev):
        _call("moe_amd_update_expert_biases", ptrs.data_ptr(), ptrs[L:].data_ptr(), L, E,
              float(update_rate), 1 if is_global else 0, float(alpha) if is_global else 0.0,
              stats.data_ptr(), _stream(biases[0]))
    v = stats.cpu().tolist()
    return {"routing/expert_bias_mean": v[0], "routing/expert_bias_std": v[1],
            "routing/expert_bias_min": v[2], "routing/expert_bias_max": v[3]}
