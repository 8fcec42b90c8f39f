"""Pins the CPU oracle (oracle/moe_oracle.py) against closed forms, brute
force, hand-derived known answers and the properties the reference's own
router tests assert (tests/test_router_deepseek_v3.py).  CPU only."""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as O


def _brute_topk(row, k):
    return sorted(range(len(row)), key=lambda e: (-row[e], e))[:k]


# ---------------------------------------------------------------- top-k

def test_rank_topk_known_answer():
    v = torch.tensor([[1.0, 3.0, 3.0, 2.0, 3.0], [0.0, -0.0, 5.0, 5.0, -1.0]])
    vals, idx = O.rank_topk(v, 3)
    # hand-derived: ties resolve to the lower index; -0.0 == 0.0
    assert idx.tolist() == [[1, 2, 4], [2, 3, 0]]
    assert vals.tolist() == [[3.0, 3.0, 3.0], [5.0, 5.0, 0.0]]


def test_rank_topk_nan_and_signed_zero_known_answer():
    """torch.topk places NaN above every number (either sign bit); NaNs among
    themselves and -0 / +0 keep index order (hand-derived)."""
    nan = float("nan")
    v = torch.tensor([[1.0, nan, 3.0, -0.0, 0.0, float("inf"), -nan, -2.0]])
    vals, idx = O.rank_topk(v, 8)
    assert idx.tolist() == [[1, 6, 5, 2, 0, 3, 4, 7]]
    # softmax router: a NaN logit makes the whole prob row NaN -> all entries
    # tie -> the K lowest indices
    logits = torch.tensor([[0.5, 2.0, nan, -1.0, 3.0, 0.0]])
    p, w, i = O.softmax_router(logits, 3)
    assert torch.isnan(p).all() and i.tolist() == [[0, 1, 2]] and torch.isnan(w).all()
    # sigmoid router: only that score is NaN, and it ranks first
    s, w, i = O.sigmoid_router(logits, None, 3)
    assert i.tolist() == [[2, 4, 1]]


def test_rank_topk_brute_force_with_ties():
    g = torch.Generator().manual_seed(1)
    v = torch.randint(0, 4, (200, 9), generator=g).float()
    for k in (1, 3, 9):
        _, idx = O.rank_topk(v, k)
        for t in range(v.shape[0]):
            assert idx[t].tolist() == _brute_topk(v[t].tolist(), k)


# -------------------------------------------------------------- routers

def test_softmax_router_closed_form():
    g = torch.Generator().manual_seed(2)
    logits = torch.randn(64, 16, generator=g, dtype=torch.float64)
    probs, w, idx = O.softmax_router(logits.to(torch.bfloat16), 4)
    z = logits.to(torch.bfloat16).double()
    p = torch.exp(z - z.max(-1, keepdim=True).values)
    p = p / p.sum(-1, keepdim=True)
    assert torch.allclose(probs.double(), p, rtol=1e-6, atol=1e-9)
    for t in range(64):
        assert idx[t].tolist() == _brute_topk(p[t].tolist(), 4)
    v = p.gather(1, idx)
    assert torch.allclose(w.double(), v / v.sum(-1, keepdim=True), rtol=1e-6)
    assert torch.allclose(w.sum(-1).double(), torch.ones(64, dtype=torch.float64), atol=1e-6)


def test_softmax_router_offset_and_no_renorm():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(32, 8, generator=g)
    off = torch.linspace(-1, 1, 8)
    probs, w, idx = O.softmax_router(logits, 2, renormalize=False, logit_offset=off)
    p = torch.softmax(logits + off, -1)
    assert torch.allclose(probs, p, atol=1e-7)
    assert torch.equal(w, p.gather(1, idx))


def test_softmax_router_ties_known_answer():
    # Four experts with equal logits: a stable ranking keeps expert order.
    logits = torch.tensor([[0.5, 0.5, 0.5, 0.5], [0.1, 0.7, 0.7, -2.0]])
    _, w, idx = O.softmax_router(logits, 2)
    assert idx.tolist() == [[0, 1], [1, 2]]
    assert torch.allclose(w, torch.full((2, 2), 0.5))


def _megatron_sigmoid(logits, bias, k, sf):
    """The reference test's Megatron replica (test_router_deepseek_v3.py:359-373),
    restated: sigmoid fp32, biased top-k, unbiased gather, /(sum+1e-20), *sf."""
    scores = torch.sigmoid(logits.float())
    _, idx = torch.topk(scores + bias.float(), k=k, dim=-1)
    gathered = torch.gather(scores, 1, idx)
    probs = gathered / (gathered.sum(-1, keepdim=True) + 1e-20) * sf
    return scores, probs, idx


def test_sigmoid_router_matches_megatron_replica():
    g = torch.Generator().manual_seed(999)
    logits = torch.randn(64, 16, generator=g) * 0.7
    bias = torch.randn(16, generator=g) * 0.01
    scores, w, idx = O.sigmoid_router(logits, bias, 4, True, 2.5)
    s_ref, p_ref, i_ref = _megatron_sigmoid(logits, bias, 4, 2.5)
    assert torch.equal(idx, i_ref)
    assert torch.allclose(w, p_ref, atol=1e-5)
    assert torch.equal(scores, s_ref)


def test_sigmoid_router_reference_properties():
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(8, 32, generator=g)
    _, w, _ = O.sigmoid_router(logits, None, 4, True, 2.5)
    assert torch.allclose(w.sum(-1), torch.full((8,), 2.5), atol=1e-4)
    # no NaN with sigmoid ~ 0 (test_router_deepseek_v3.py:110-120)
    _, w0, _ = O.sigmoid_router(torch.full((4, 16), -6400.0), None, 4, True, None)
    assert not torch.isnan(w0).any() and not torch.isinf(w0).any()
    # bf16 weights are the fp32 values rounded once
    _, wb, _ = O.sigmoid_router(logits, None, 4, True, 2.5, weights_dtype=torch.bfloat16)
    assert torch.equal(wb, w.to(torch.bfloat16))


def test_sigmoid_router_bf16_scores_known_answers():
    """The router's lines evaluated on bf16 scores (the reference under bf16
    autocast): hand-derived values."""
    # renormalisation in bf16: 0.5 / 0.75 and 0.25 / 0.75 each rounded to
    # 8 significant bits (1.0101011b x 2^-1 and x 2^-2); they sum to 1.0019531
    s = torch.tensor([[0.5, 0.25, 0.125, 0.0625]], dtype=torch.bfloat16)
    w, idx = O.sigmoid_router_from_scores(s, None, 2, True, None, weights_dtype=torch.float32)
    assert idx.tolist() == [[0, 1]]
    assert w.tolist() == [[0.66796875, 0.333984375]]
    w32, _ = O.sigmoid_router_from_scores(s.float(), None, 2, True, None)
    assert torch.allclose(w32, torch.tensor([[2 / 3, 1 / 3]]))
    assert w32.tolist() != w.tolist()
    # scores are rounded before the bias is added: 0.75 + 2^-12 and 0.75 are
    # one bf16 value, so the 2^-14 bias of expert 1 decides; in fp32 expert 0
    # stays ahead by 2^-12 - 2^-14
    s32 = torch.tensor([[0.75 + 2.0 ** -12, 0.75]])
    bias = torch.tensor([0.0, 2.0 ** -14])
    _, i32 = O.sigmoid_router_from_scores(s32, bias, 1, True)
    _, i16 = O.sigmoid_router_from_scores(s32.to(torch.bfloat16), bias, 1, True)
    assert i32.tolist() == [[0]] and i16.tolist() == [[1]]
    # bf16 logits keep bf16 scores (torch.sigmoid leaves the dtype)
    sc, _, _ = O.sigmoid_router(torch.zeros(2, 8, dtype=torch.bfloat16), None, 2)
    assert sc.dtype == torch.bfloat16 and torch.equal(sc.float(), torch.full((2, 8), 0.5))


def test_group_limited_topk_constraints():
    g = torch.Generator().manual_seed(42)
    scores = torch.randn(128, 32, generator=g).abs()
    vals, idx = O.group_limited_topk(scores, 8, 8, 4)
    assert idx.shape == (128, 8)
    groups = (idx // 4)
    for t in range(128):
        assert len(set(groups[t].tolist())) <= 4
    # brute force: the kept groups are the 4 best by top-2 sums
    for t in range(16):
        gs = [sorted(scores[t, 4 * q:4 * q + 4].tolist(), reverse=True)[:2] for q in range(8)]
        gsum = [a + b for a, b in gs]
        keep = set(_brute_topk(gsum, 4))
        allowed = [e for e in range(32) if e // 4 in keep]
        exp = sorted(allowed, key=lambda e: (-scores[t, e].item(), e))[:8]
        assert idx[t].tolist() == exp
    _, flat = O.rank_topk(scores, 8)
    assert not torch.equal(flat, idx)


def test_router_backward_formulas_match_autograd():
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(16, 12, generator=g, dtype=torch.float64, requires_grad=True)
    probs = torch.softmax(logits, -1)
    _, idx = O.rank_topk(probs.detach(), 3)
    v = probs.gather(1, idx)
    w = v / v.sum(-1, keepdim=True)
    dw = torch.randn(16, 3, generator=g, dtype=torch.float64)
    dp = torch.randn(16, 12, generator=g, dtype=torch.float64)
    (gl,) = torch.autograd.grad((w * dw).sum() + (probs * dp).sum(), logits)
    mine = O.softmax_router_backward(probs.detach(), idx, dw, dp, True, torch.float64)
    assert torch.allclose(mine, gl, atol=1e-12)

    lg = torch.randn(16, 12, generator=g, dtype=torch.float64, requires_grad=True)
    s = torch.sigmoid(lg)
    bias = torch.randn(12, generator=g, dtype=torch.float64) * 0.1
    _, idx2 = O.rank_topk((s + bias).detach(), 3)
    v2 = s.gather(1, idx2)
    w2 = v2 / (v2.sum(-1, keepdim=True) + 1e-20) * 2.5
    (g2,) = torch.autograd.grad((w2 * dw).sum() + (s * dp).sum(), lg)
    mine2 = O.sigmoid_router_backward(s.detach(), idx2, dw, dp, True, 2.5)
    assert torch.allclose(mine2.double(), g2, atol=1e-6)


# ---------------------------------------------------------- permutation

def _brute_permute(ids, E):
    buckets = [[] for _ in range(E + 1)]
    for s, e in enumerate(ids):
        buckets[e if 0 <= e < E else E].append(s)
    row_src = [s for b in buckets for s in b]
    counts = [len(b) for b in buckets[:E]]
    return row_src, counts


@pytest.mark.parametrize("T,K,E,sentinels", [(37, 4, 16, False), (300, 8, 128, False),
                                              (64, 2, 8, True), (5, 1, 1, False)])
def test_permute_brute_force(T, K, E, sentinels):
    g = torch.Generator().manual_seed(T * 31 + E)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    if sentinels:
        idx[::3, 0] = E + 2   # expert-parallel style sentinel ids
    plan = O.permute(idx, E)
    row_src, counts = _brute_permute(idx.reshape(-1).tolist(), E)
    assert plan.row_src.tolist() == row_src
    assert plan.counts.tolist() == counts
    assert plan.offsets.tolist() == [0] + list(itertools.accumulate(counts))
    assert plan.slot[plan.row_src].tolist() == list(range(T * K))
    for b, bm in enumerate(O.TILE_SIZES):
        exp = [0] + list(itertools.accumulate((c + bm - 1) // bm for c in counts))
        assert plan.tile_starts[b].tolist() == exp


# --------------------------------------------------------------- experts

def _experts_inputs(T, H, E, K, I, dtype, seed=0, sentinels=False, bf16_weights=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g)
    wr = torch.randn(E, H, generator=g) * 0.02
    w1 = torch.randn(E, 2 * I, H, generator=g) * 0.02
    w2 = torch.randn(E, H, I, generator=g) * 0.02
    probs, w, idx = O.softmax_router(x @ wr.T, K)
    if sentinels:
        idx = idx.clone()
        idx[::5, -1] = E
    if bf16_weights:
        w = w.to(torch.bfloat16)
    return x.to(dtype), idx, w, w1.to(dtype), w2.to(dtype)


@pytest.mark.parametrize("sentinels", [False, True])
def test_experts_forward_matches_eager_fp64(sentinels):
    x, idx, w, w1, w2 = _experts_inputs(48, 32, 6, 2, 16, torch.float64, sentinels=sentinels)
    out, _ = O.experts_forward(x, idx, w.double(), w1, w2)
    ref = O.experts_eager(x, idx, w.double(), w1, w2)
    assert torch.allclose(out, ref, rtol=1e-10, atol=1e-12)


def test_experts_backward_matches_autograd_fp64():
    x, idx, w, w1, w2 = _experts_inputs(40, 32, 5, 2, 16, torch.float64)
    w = w.double()
    leaves = [t.clone().requires_grad_(True) for t in (x, w, w1, w2)]
    ref = O.experts_eager(leaves[0], idx, leaves[1], leaves[2], leaves[3])
    g = torch.Generator().manual_seed(7)
    dout = torch.randn(ref.shape, generator=g, dtype=torch.float64)
    grads = torch.autograd.grad((ref * dout).sum(), leaves)
    out, cache = O.experts_forward(x, idx, w, w1, w2)
    dx, dw, dw1, dw2, _ = O.experts_backward(cache, x, w, w1, w2, dout)
    for mine, theirs in zip((dx, dw, dw1, dw2), grads):
        assert torch.allclose(mine, theirs, rtol=1e-9, atol=1e-11)


def test_experts_bf16_within_tolerance_of_fp64():
    x, idx, w, w1, w2 = _experts_inputs(64, 64, 8, 2, 64, torch.bfloat16, seed=4)
    out, _ = O.experts_forward(x, idx, w, w1, w2)
    ref = O.experts_eager(x.double(), idx, w.double(), w1.double(), w2.double())
    err = (out.double() - ref).abs().max() / ref.abs().max()
    assert err < 2e-2


def test_experts_empty_experts_get_zero_weight_grads():
    x, idx, w, w1, w2 = _experts_inputs(16, 32, 6, 1, 16, torch.float64)
    idx = torch.where(idx == 3, torch.zeros_like(idx), idx)  # expert 3 unused
    out, cache = O.experts_forward(x, idx, w.double(), w1, w2)
    _, _, dw1, dw2, _ = O.experts_backward(cache, x, w.double(), w1, w2, torch.ones_like(out))
    assert dw1[3].abs().max() == 0 and dw2[3].abs().max() == 0


def test_planted_mistake_is_caught():
    """A plausible slip (gate and up swapped) must fail the fp64 eager pin."""
    x, idx, w, w1, w2 = _experts_inputs(24, 32, 4, 2, 16, torch.float64)
    I = w1.shape[1] // 2
    swapped = torch.cat([w1[:, I:], w1[:, :I]], dim=1)
    out, _ = O.experts_forward(x, idx, w.double(), swapped, w2)
    ref = O.experts_eager(x, idx, w.double(), w1, w2)
    assert not torch.allclose(out, ref, rtol=1e-6)
