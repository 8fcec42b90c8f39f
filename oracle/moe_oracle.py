"""CPU oracle for the MoE expert-layer path — TEST INFRASTRUCTURE ONLY.

A plain restatement (torch on the CPU, numpy for the integer work) of the
reference algorithm for the hot path.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may use
it, and only as the checker / the timed CPU baseline; the product package
``moe_amd`` never imports it and has no CPU fallback.

Reference (leonmodal/moe, transformers 5.x grouped_mm backend):
  softmax router      src/models/modeling_qwen3_moe.py:266-275
  DeepSeek router     src/models/router.py:103-155, group_limited_topk :22-70
  permutation         transformers/integrations/moe.py:389-403 (sort, histc, cumsum)
  grouped GEMM 1      transformers/integrations/moe.py:439-442 (-> _grouped_mm :308-336)
  SwiGLU              transformers/integrations/moe.py:446-447, :509-520
  grouped GEMM 2      transformers/integrations/moe.py:453-459
  combine             transformers/integrations/moe.py:461-478
  backward formulas   transformers/integrations/moe.py:226-242 (per-expert dX/dW)
  eager experts loop  src/models/modeling_qwen3_moe.py:230-254 (second, dense oracle)

Rounding points reproduced for bf16 (the reference's tensors are bf16 at
these points): each grouped GEMM output, silu(gate), silu*up, the weighted
rows when the routing weights are bf16; the combine sums over K in fp32 in k
order and rounds once.  In fp32/fp64 every cast is the identity.

How each function is pinned (tests/test_oracle.py):
  rank_topk            brute force over all orderings on small rows; crafted
                       ties with hand-derived answers
  softmax_router       closed form exp/sum in fp64; reference test
                       properties (weights sum to 1)
  sigmoid_router       the reference tests' Megatron replica and properties
                       (tests/test_router_deepseek_v3.py:142-190, 197-267,
                       331-422) restated; group constraint
  permute              pure-Python counting sort; invariants (bijection,
                       sorted keys, stable, offsets = cumsum(counts))
  experts_forward      eager per-token dense loop in fp64 (reference a14 form)
  experts_backward     torch.autograd of the fp64 eager loop
  router backwards     torch.autograd of the fp64 router restatements
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

TILE_SIZES = (64, 128, 256)


# ------------------------------------------------------------------ top-k

def rank_topk(values: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k along the last dim, sorted descending; equal values keep the
    lower index first (a stable sort of -values; -0 == +0).  A NaN ranks
    above every number, as torch.topk places it, NaNs among themselves by
    index.  Returns (values, index)."""
    v = values.detach().cpu().numpy()
    nan = np.isnan(v)
    # lexsort: last key is primary; both sorts are stable
    order = np.lexsort((np.where(nan, 0.0, -v), ~nan), axis=-1)[..., :k]
    idx = torch.from_numpy(np.ascontiguousarray(order)).to(torch.int64)
    return torch.gather(values.cpu(), -1, idx), idx


# ----------------------------------------------------------------- routers

def softmax_router(logits: torch.Tensor, top_k: int, renormalize: bool = True,
                   logit_offset: torch.Tensor | None = None):
    """Qwen3MoeTopKRouter after its F.linear (modeling_qwen3_moe.py:269-274):
    probs = softmax(logits, fp32); top-k; w /= w.sum() (no epsilon).
    Returns (probs [T,E] fp32, weights [T,K] fp32, index [T,K] int64)."""
    z = logits.float()
    if logit_offset is not None:
        z = z + logit_offset.float()
    probs = torch.softmax(z, dim=-1)
    w, idx = rank_topk(probs, top_k)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return probs, w.to(torch.float32), idx


def group_limited_topk(scores: torch.Tensor, top_k: int, num_groups: int, group_topk: int):
    """router.py:22-70: groups scored by the sum of their top (K/group_topk)
    scores, group_topk groups kept, top-k over the kept experts."""
    T, E = scores.shape
    eg = E // num_groups
    per = top_k // group_topk
    gvals, _ = rank_topk(scores.view(T, num_groups, eg), per)
    gscore = gvals.sum(dim=-1)
    _, gidx = rank_topk(gscore, group_topk)
    gmask = torch.zeros(T, num_groups, dtype=torch.bool)
    gmask.scatter_(1, gidx, True)
    emask = gmask.unsqueeze(-1).expand(T, num_groups, eg).reshape(T, E)
    masked = scores.masked_fill(~emask, float("-inf"))
    return rank_topk(masked, top_k)


def sigmoid_router(logits: torch.Tensor, expert_bias: torch.Tensor | None, top_k: int,
                   renormalize: bool = True, scaling_factor: float | None = None,
                   num_groups: int | None = None, group_topk: int | None = None,
                   weights_dtype: torch.dtype = torch.float32):
    """DeepSeekRouter after its gating linear (router.py:111-140).  fp32
    logits: the fp32 path.  bf16 logits: the same lines as torch runs them
    under bf16 autocast (whose F.linear(h.float(), W.float()) returns bf16):
    torch.sigmoid keeps bf16 (:112).  Returns (scores [T,E] in the logits'
    floating dtype (fp32 unless bf16), weights [T,K] weights_dtype, index
    int64)."""
    lp = logits.dtype == torch.bfloat16
    scores = torch.sigmoid(logits if lp else logits.float())
    w, idx = sigmoid_router_from_scores(scores, expert_bias, top_k, renormalize, scaling_factor,
                                        num_groups, group_topk, weights_dtype)
    return scores, w, idx


def sigmoid_router_from_scores(scores: torch.Tensor, expert_bias: torch.Tensor | None,
                               top_k: int, renormalize: bool = True,
                               scaling_factor: float | None = None,
                               num_groups: int | None = None, group_topk: int | None = None,
                               weights_dtype: torch.dtype = torch.float32):
    """router.py:114-140 on given scores, in the scores' dtype as torch
    evaluates those lines: the biased scores fp32 (scores + fp32 bias, :116),
    the gathered weights, their sum (+1e-20), quotient and scaling in the
    scores' dtype (bf16 for bf16 scores).  Returns (weights, index)."""
    biased = scores.float() + (expert_bias.float() if expert_bias is not None else 0.0)
    if num_groups is not None and group_topk is not None:
        _, idx = group_limited_topk(biased, top_k, num_groups, group_topk)
    else:
        _, idx = rank_topk(biased, top_k)
    w = scores.gather(1, idx)
    if renormalize:
        w = w / (w.sum(dim=-1, keepdim=True) + 1e-20)
    if scaling_factor:
        w = w * scaling_factor
    return w.to(weights_dtype), idx


def softmax_router_backward(probs, idx, d_w, d_probs, renormalize: bool, logits_dtype):
    """Autograd of softmax -> gather -> renorm, written out:
    dv_k = g_k/S - sum_j g_j v_j / S^2; dp = d_probs + scatter(dv);
    dlogits = p * (dp - sum(p * dp))."""
    p = probs.double()
    v = p.gather(1, idx)
    g = d_w.double()
    if renormalize:
        s = v.sum(-1, keepdim=True)
        dv = g / s - (g * v).sum(-1, keepdim=True) / (s * s)
    else:
        dv = g
    dp = torch.zeros_like(p) if d_probs is None else d_probs.double().clone()
    dp.scatter_add_(1, idx, dv)
    dl = p * (dp - (p * dp).sum(-1, keepdim=True))
    return dl.to(logits_dtype)


def sigmoid_router_backward(scores, idx, d_w, d_scores, renormalize: bool,
                            scaling_factor: float | None):
    """Autograd of sigmoid -> gather -> renorm(+1e-20) -> scale, written out."""
    y = scores.double()
    v = y.gather(1, idx)
    g = d_w.double()
    if scaling_factor:
        g = g * scaling_factor
    if renormalize:
        s = v.sum(-1, keepdim=True) + 1e-20
        dv = g / s - (g * v).sum(-1, keepdim=True) / (s * s)
    else:
        dv = g
    ds = torch.zeros_like(y) if d_scores is None else d_scores.double().clone()
    ds.scatter_add_(1, idx, dv)
    return (ds * y * (1 - y)).float()


# ------------------------------------------------------------- permutation

@dataclass
class Plan:
    counts: np.ndarray      # [E]
    offsets: np.ndarray     # [E+1] exclusive; offsets[E] = rows of real experts
    row_src: np.ndarray     # [S] sorted row -> flat t*K+k
    slot: np.ndarray        # [S] flat -> sorted row
    tile_starts: np.ndarray # [3, E+1]


def permute(topk_index: torch.Tensor, num_experts: int) -> Plan:
    """Stable counting sort of the flat routed ids (moe.py:389-403 with a
    stable sort); ids outside [0,E) form a trailing sentinel bin."""
    ids = topk_index.reshape(-1).cpu().numpy().astype(np.int64)
    E = int(num_experts)
    keys = np.where((ids >= 0) & (ids < E), ids, E)
    row_src = np.argsort(keys, kind="stable").astype(np.int32)
    slot = np.empty_like(row_src)
    slot[row_src] = np.arange(row_src.size, dtype=np.int32)
    binc = np.bincount(keys, minlength=E + 1).astype(np.int64)
    counts = binc[:E].astype(np.int32)
    offsets = np.zeros(E + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(binc[:E])
    ts = np.zeros((len(TILE_SIZES), E + 1), dtype=np.int32)
    for b, bm in enumerate(TILE_SIZES):
        ts[b, 1:] = np.cumsum((counts.astype(np.int64) + bm - 1) // bm)
    return Plan(counts, offsets, row_src, slot, ts)


# ---------------------------------------------------------------- experts

def _round(t: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    return t.to(dt).to(torch.float32 if dt != torch.float64 else torch.float64)


def _acc_dtype(dt: torch.dtype) -> torch.dtype:
    return torch.float64 if dt == torch.float64 else torch.float32


def experts_forward(x: torch.Tensor, topk_index: torch.Tensor, topk_weights: torch.Tensor,
                    gate_up_proj: torch.Tensor, down_proj: torch.Tensor):
    """grouped_mm_experts_forward (moe.py:377-478) on the CPU.

    Returns (out [T,H] in x.dtype, cache) where cache holds the plan and the
    intermediates (xs, gate_up, act, y, in the weights' dtype) the backward
    and the per-kernel parity tests use."""
    dt = gate_up_proj.dtype
    acc = _acc_dtype(dt)
    T, H = x.shape
    K = topk_index.shape[1]
    E, I2, _ = gate_up_proj.shape
    I = I2 // 2
    plan = permute(topk_index, E)
    off = plan.offsets
    row_src = torch.from_numpy(plan.row_src.astype(np.int64))
    slot = torch.from_numpy(plan.slot.astype(np.int64))
    S = T * K
    xs = x.to(dt)[row_src // K]
    W1 = gate_up_proj.to(acc)
    W2 = down_proj.to(acc)
    gu = torch.zeros(S, I2, dtype=acc)
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            gu[a:b] = xs[a:b].to(acc) @ W1[e].T
    gu = _round(gu, dt)
    g, u = gu[:, :I], gu[:, I:]
    s = _round(F.silu(g), dt)
    act = _round(s * u, dt)
    y = torch.zeros(S, H, dtype=acc)
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            y[a:b] = act[a:b] @ W2[e].T
    y = _round(y, dt)
    wg = topk_weights.reshape(-1)[row_src].to(acc)
    z = y * wg[:, None]
    if topk_weights.dtype == dt and dt != acc:
        z = _round(z, dt)  # bf16 weights: bf16 * bf16 product is a bf16 tensor
    z[int(off[E]):] = 0.0  # EP sentinel rows contribute nothing (moe.py:464-465)
    zt = z[slot].view(T, K, H)
    out = zt[:, 0].clone()
    for k in range(1, K):
        out = out + zt[:, k]
    cache = dict(plan=plan, xs=xs, gate_up=gu.to(dt), act=act.to(dt), y=y.to(dt),
                 dtype=dt, top_k=K)
    return out.to(x.dtype), cache


def experts_backward(cache: dict, x: torch.Tensor, topk_weights: torch.Tensor,
                     gate_up_proj: torch.Tensor, down_proj: torch.Tensor, d_out: torch.Tensor):
    """Backward of experts_forward at the reference's autograd rounding points.
    Returns (d_x, d_topk_weights, d_gate_up_proj, d_down_proj)."""
    dt = cache["dtype"]
    acc = _acc_dtype(dt)
    plan: Plan = cache["plan"]
    K = cache["top_k"]
    T, H = x.shape
    E, I2, _ = gate_up_proj.shape
    I = I2 // 2
    off = plan.offsets
    nvalid = int(off[E])
    row_src = torch.from_numpy(plan.row_src.astype(np.int64))
    slot = torch.from_numpy(plan.slot.astype(np.int64))
    tok = row_src // K
    y = cache["y"].to(acc)
    act = cache["act"].to(acc)
    gu = cache["gate_up"].to(acc)
    xs = cache["xs"].to(acc)
    W1 = gate_up_proj.to(acc)
    W2 = down_proj.to(acc)
    wg = topk_weights.reshape(-1)[row_src].to(acc)
    g_rows = d_out.to(acc)[tok]
    # combine backward
    dy = _round(g_rows * wg[:, None], dt)
    prod = g_rows * y
    if topk_weights.dtype == dt and dt != acc:
        dwg = _round(_round(prod, dt).sum(-1), dt)
    else:
        dwg = prod.sum(-1)
    dy[nvalid:] = 0.0
    dwg[nvalid:] = 0.0
    d_w = torch.zeros(T * K, dtype=acc)
    d_w[row_src] = dwg
    d_w = d_w.view(T, K).to(topk_weights.dtype)
    # GEMM-2 backward
    da = torch.zeros(T * K, I, dtype=acc)
    dW2 = torch.zeros(E, H, I, dtype=acc)
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            da[a:b] = dy[a:b] @ W2[e]
            dW2[e] = dy[a:b].T @ act[a:b]
    da = _round(da, dt)
    # SwiGLU backward (silu backward: dy * sig * (1 + x * (1 - sig)))
    g, u = gu[:, :I], gu[:, I:]
    sg = torch.sigmoid(g)
    s = _round(F.silu(g), dt)
    ds = _round(da * u, dt)
    du = _round(da * s, dt)
    dg = _round(ds * (sg * (1 + g * (1 - sg))), dt)
    dgu = torch.cat([dg, du], dim=-1)
    # GEMM-1 backward
    dxs = torch.zeros(T * K, H, dtype=acc)
    dW1 = torch.zeros(E, I2, H, dtype=acc)
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            dxs[a:b] = dgu[a:b] @ W1[e]
            dW1[e] = dgu[a:b].T @ xs[a:b]
    dxs = _round(dxs, dt)
    dxs[nvalid:] = 0.0
    # gather backward: sum over the K routed copies of each token, k order
    dxt = dxs[slot].view(T, K, H)
    d_x = dxt[:, 0].clone()
    for k in range(1, K):
        d_x = d_x + dxt[:, k]
    return d_x.to(x.dtype), d_w, dW1.to(dt), dW2.to(dt), dict(d_y=dy.to(dt), d_gate_up=dgu.to(dt),
                                                               d_xs=dxs.to(dt))


def experts_eager(x, topk_index, topk_weights, gate_up_proj, down_proj):
    """Dense per-token form of the expert layer (the reference's eager loop,
    modeling_qwen3_moe.py:230-254) built from differentiable torch ops; used
    in fp64 to pin experts_forward and, through autograd, experts_backward."""
    T, H = x.shape
    K = topk_index.shape[1]
    E, I2, _ = gate_up_proj.shape
    I = I2 // 2
    out = torch.zeros_like(x)
    for e in range(E):
        tok, kk = torch.where(topk_index == e)
        if tok.numel() == 0:
            continue
        h = x[tok]
        gu = h @ gate_up_proj[e].T
        a = F.silu(gu[:, :I]) * gu[:, I:]
        yv = a @ down_proj[e].T
        out = out.index_add(0, tok, yv * topk_weights[tok, kk, None])
    return out
