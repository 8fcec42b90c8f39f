"""Pins of the routing-consumer oracle (oracle/balancing_oracle.py) against
facts it does not restate: the reference tests' closed forms, the DeepSeek-V3
paper and Megatron-LM formulations, invariances, and finite differences.
CPU only."""
from __future__ import annotations

import math

import pytest
import torch

from oracle import balancing_oracle as B


def _rand_probs(T, E, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.softmax(torch.randn(T, E, generator=g, dtype=torch.float64), dim=-1)


# ------------------------------------------------------------ Switch loss

def test_switch_uniform_gives_top_k():
    """tests/test_aux_loss_fix.py:9-14: uniform probabilities give top_k."""
    probs = torch.ones(1000, 128) / 128
    loss = B.switch_aux_loss((probs,), 128, 4)
    assert abs(loss.item() - 4.0) < 1e-9


def test_switch_skew_bounds():
    """tests/test_aux_loss_fix.py:17-35: 4 hot experts >> 20, 16 hot > 6."""
    p = torch.ones(1000, 128) * 0.001
    p[:, :4] = 0.25
    p = p / p.sum(-1, keepdim=True)
    assert B.switch_aux_loss((p,), 128, 4).item() > 20.0
    p = torch.ones(1000, 128) * 0.005
    p[:, :16] = 0.05
    p = p / p.sum(-1, keepdim=True)
    assert B.switch_aux_loss((p,), 128, 4).item() > 6.0


def test_switch_collapsed_gives_num_experts():
    """All mass on experts 0..K-1 (1/K each): every token selects them, so
    f_i = 1 and p_i = 1/K for i < K: loss = E * K * (1/K) = E."""
    E, K = 32, 4
    p = torch.zeros(100, E, dtype=torch.float64)
    p[:, :K] = 1.0 / K
    assert abs(B.switch_aux_loss((p,), E, K).item() - E) < 1e-12


def test_switch_mask_equals_dropping_tokens():
    """A 0/1 attention mask is the same as removing the masked tokens."""
    bsz, S, E, K = 2, 40, 16, 2
    probs = _rand_probs(bsz * S, E, 1)
    mask = torch.ones(bsz, S)
    mask[0, 30:] = 0
    mask[1, :7] = 0
    keep = mask.reshape(-1).bool()
    two = (probs, _rand_probs(bsz * S, E, 2))
    a = B.switch_aux_loss(two, E, K, attention_mask=mask)
    b = B.switch_aux_loss(tuple(x[keep] for x in two), E, K)
    assert abs(a.item() - b.item()) < 1e-12


def test_switch_gradient_finite_differences():
    E, K = 8, 2
    probs = _rand_probs(30, E, 3).requires_grad_(True)
    loss = B.switch_aux_loss((probs,), E, K)
    (g,) = torch.autograd.grad(loss, probs)
    h = 1e-6
    for t, e in [(0, 0), (5, 3), (29, 7)]:
        d = torch.zeros_like(probs)
        d[t, e] = h
        with torch.no_grad():  # the selection does not move for a step this small
            num = (B.switch_aux_loss((probs + d,), E, K) - B.switch_aux_loss((probs - d,), E, K))
        assert abs(num.item() / (2 * h) - g[t, e].item()) < 1e-6


# -------------------------------------------------- sequence-wise loss

def _paper_seq_loss(raw_logits, E, K, bsz):
    """DeepSeek-V3 Eqs. 17-20 (restated from tests/test_seq_loss_vs_paper.py:
    24-57): selection on the raw sigmoid, P on the normalised scores, per
    sequence, written as an explicit loop over sequences and tokens."""
    total = 0.0
    for raw in raw_logits:
        T = raw.shape[0]
        S = T // bsz
        s = torch.sigmoid(raw.double())
        per_seq = []
        for b in range(bsz):
            f = [0.0] * E
            P = [0.0] * E
            for t in range(b * S, (b + 1) * S):
                row = s[t]
                den = float(row.sum()) + 1e-20
                for e in row.argsort(descending=True, stable=True)[:K].tolist():
                    f[e] += E / (K * S)
                for e in range(E):
                    P[e] += float(row[e]) / den / S
            per_seq.append(sum(f[e] * P[e] for e in range(E)))
        total += sum(per_seq) / bsz
    return total / len(raw_logits)


def _megatron_seq_loss_b1(raw_logits, E, K):
    """Megatron-LM's switch_load_balancing_loss_func on one sequence
    (restated from tests/test_seq_loss_vs_paper.py:60-101, batch 1)."""
    total = 0.0
    for raw in raw_logits:
        S = raw.shape[0]
        sc = torch.sigmoid(raw.double())
        sc = sc / (sc.sum(-1, keepdim=True) + 1e-20)
        top = sc.topk(K, dim=-1).indices
        routing = torch.zeros_like(sc).scatter(1, top, 1.0)
        total += float((sc.sum(0) * routing.sum(0)).sum()) * E / (K * S * S)
    return total / len(raw_logits)


def test_seq_matches_paper_formulation():
    bsz, S, E, K = 3, 24, 16, 4
    g = torch.Generator().manual_seed(42)
    raw = [torch.randn(bsz * S, E, generator=g, dtype=torch.float64) for _ in range(2)]
    ours = B.seq_aux_loss(tuple(torch.sigmoid(r) for r in raw), E, K, batch_size=bsz).item()
    assert abs(ours - _paper_seq_loss(raw, E, K, bsz)) < 1e-12


def test_seq_matches_megatron_single_sequence():
    S, E, K = 64, 32, 8
    g = torch.Generator().manual_seed(7)
    raw = [torch.randn(S, E, generator=g, dtype=torch.float64) for _ in range(3)]
    ours = B.seq_aux_loss(tuple(torch.sigmoid(r) for r in raw), E, K, batch_size=1).item()
    assert abs(ours - _megatron_seq_loss_b1(raw, E, K)) < 1e-12


def test_seq_balanced_routing_gives_one():
    """Uniform scores and exactly balanced selections: f_i = 1, P_i = 1/E."""
    E, K, S = 8, 2, 16
    scores = torch.full((S, E), 0.3, dtype=torch.float64)
    sel = torch.tensor([[(2 * t) % E, (2 * t + 1) % E] for t in range(S)])
    loss = B.seq_aux_loss((scores,), E, K, batch_size=1, selected_experts=(sel,))
    assert abs(loss.item() - 1.0) < 1e-12


def test_seq_gradient_finite_differences():
    E, K, bsz, S = 8, 2, 2, 10
    g = torch.Generator().manual_seed(5)
    s = torch.sigmoid(torch.randn(bsz * S, E, generator=g, dtype=torch.float64)).requires_grad_(True)
    sel = torch.randint(0, E, (bsz * S, K), generator=g)
    loss = B.seq_aux_loss((s,), E, K, batch_size=bsz, selected_experts=(sel,))
    (gr,) = torch.autograd.grad(loss, s)
    h = 1e-6
    for t, e in [(0, 0), (7, 5), (19, 7)]:
        d = torch.zeros_like(s)
        d[t, e] = h
        with torch.no_grad():
            num = (B.seq_aux_loss((s + d,), E, K, bsz, (sel,)) -
                   B.seq_aux_loss((s - d,), E, K, bsz, (sel,)))
        assert abs(num.item() / (2 * h) - gr[t, e].item()) < 1e-8


# ------------------------------------------------------ routing stats

def test_stats_uniform_and_collapsed():
    """tests/test_routing_stats.py:32-81 closed forms (the reference file's
    keys that its code no longer emits, e.g. utilization, are not used)."""
    uni = B.routing_stats([torch.full((64, 8), 1.0 / 8)], 2)
    assert uni["routing/layer_00_load_imbalance"] == pytest.approx(4.0)  # ties: experts 0,1
    col = torch.zeros(32, 8)
    col[:, 0] = 1.0
    st = B.routing_stats([col], 1)
    assert st["routing/layer_00_load_imbalance"] == pytest.approx(8.0)
    assert st["routing/layer_00_entropy"] < 0.01
    assert st["routing/layer_00_num_active_experts"] == 1
    assert st["routing/layer_00_top_expert"] == 0
    assert abs(sum(st["_hist/routing/layer_00_expert_load_frac"]) - 1.0) < 1e-12
    # balanced counts without ties: each token's top-2 rotates over the experts
    p = torch.full((64, 8), 0.01, dtype=torch.float64)
    for t in range(64):
        p[t, (2 * t) % 8] = 0.5
        p[t, (2 * t + 1) % 8] = 0.4
    st = B.routing_stats([p], 2)
    assert st["routing/layer_00_load_imbalance"] == pytest.approx(1.0)
    assert st["routing/layer_00_load_cv"] == pytest.approx(0.0)
    assert st["routing/layer_00_entropy"] == pytest.approx(1.0, abs=1e-6)
    assert st["routing/layer_00_router_margin_mean"] == pytest.approx(0.39)
    assert st["routing/layer_00_router_margin_min"] == pytest.approx(0.39)


def test_stats_cross_layer():
    """tests/test_routing_stats.py:103-120: identical layers give similarity
    1; disjoint halves give 0."""
    p = torch.full((32, 8), 1.0 / 8)
    st = B.routing_stats([p, p], 2, is_global=True)
    assert st["routing/cross_layer_sim_mean"] == pytest.approx(1.0)
    p1 = torch.zeros(32, 8)
    p1[:, :4] = 0.25
    p2 = torch.zeros(32, 8)
    p2[:, 4:] = 0.25
    st = B.routing_stats([p1, p2], 2, is_global=True)
    assert st["routing/cross_layer_sim_mean"] < 0.1
    assert st["routing/global_pool_num_active"] == 4  # experts 0,1 and 4,5 (ties -> lower ids)


# ---------------------------------------------------- expert-bias update

def _megatron_bias(counts, bias, rate):
    """Megatron-LM get_updated_expert_bias (restated from
    tests/test_bias_update_detailed.py:97-102)."""
    avg = counts.sum(dim=-1, keepdim=True) / counts.shape[-1]
    return bias + torch.sign(avg - counts) * rate


def test_bias_update_per_layer_matches_megatron():
    g = torch.Generator().manual_seed(0)
    counts = [torch.randint(0, 50, (16,), generator=g).float() for _ in range(3)]
    biases = [torch.randn(16, generator=g) for _ in range(3)]
    new, _ = B.update_expert_biases(counts, biases, 1e-3)
    for c, b, n in zip(counts, biases, new):
        assert torch.equal(n, _megatron_bias(c, b, 1e-3))


def test_bias_update_global_and_blend_by_hand():
    counts = [torch.tensor([4.0, 0.0, 2.0, 2.0]), torch.tensor([0.0, 4.0, 2.0, 2.0])]
    biases = [torch.zeros(4), torch.zeros(4)]
    # pooled counts [4,4,4,4]: no expert is off the mean, nothing moves
    new, st = B.update_expert_biases(counts, biases, 0.5, is_global=True)
    assert all(torch.equal(n, torch.zeros(4)) for n in new)
    assert st["routing/expert_bias_std"] == 0.0
    # blended: only the per-layer part (alpha) acts
    new, _ = B.update_expert_biases(counts, biases, 0.5, is_global=True, alpha=0.25)
    assert torch.equal(new[0], torch.tensor([-0.125, 0.125, 0.0, 0.0]))
    assert torch.equal(new[1], torch.tensor([0.125, -0.125, 0.0, 0.0]))
    # per layer
    new, st = B.update_expert_biases(counts, biases, 0.5)
    assert torch.equal(new[0], torch.tensor([-0.5, 0.5, 0.0, 0.0]))
    assert st["routing/expert_bias_min"] == -0.5 and st["routing/expert_bias_max"] == 0.5
    assert st["routing/expert_bias_std"] == pytest.approx(math.sqrt(1.0 / 7.0))
