"""Irregular shapes: a fixed, seeded sample of (T, H, E, K, I) drawn over the
ranges the entry points accept (T from 1 to a few thousand, H and I any
multiple of 64, E up to 300 with empty experts, K from 1 to 8, skewed or
flat routing, EP sentinels, fp32 or bf16 routing weights).  Each runs the
expert layer fwd+bwd against the oracle (outputs and every gradient within
the bf16 bound, untouched experts' weight gradients exactly zero) and the
two routers against the oracle (indices bit-exact)."""
from __future__ import annotations

import random

import pytest
import torch
import torch.nn.functional as F

import moe_amd  # noqa: F401
from moe_amd import ops
from moe_amd.experts import experts_forward
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 2e-2


def _cases(n=16, seed=2024):
    r = random.Random(seed)
    out = []
    for _ in range(n):
        E = r.choice([1, 2, 3, 7, 16, 33, 64, 100, 128, 257, 300])
        K = r.randint(1, min(E, 8))
        out.append((r.choice([1, 5, 63, 64, 65, 511, 777, 1500, 3001]),   # T
                    64 * r.randint(1, 24),                                # H
                    E, K,
                    64 * r.randint(1, 16),                                # I
                    r.choice([0.0, 0.0, 2.0]),                            # skew
                    r.choice([0, 0, 3]),                                  # sentinel every
                    r.choice([torch.float32, torch.bfloat16])))
    return out


CASES = _cases()


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


def _inputs(T, H, E, K, I, seed, skew, sent, wdt):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    wr = torch.randn(E, H, generator=g) * 0.02
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    logits = x.float() @ wr.T
    if skew:
        logits = logits + skew * (torch.randperm(E, generator=g).float() + 1).pow(-1.1) * 8
    _, w, idx = O.softmax_router(logits, K)
    if sent and K > 1:
        idx[::sent, -1] = E  # expert-parallel sentinels: no contribution
    dout = torch.randn(T, H, generator=g).to(torch.bfloat16)
    return x, idx, w.to(wdt), w1, w2, dout


@pytest.mark.parametrize("T,H,E,K,I,skew,sent,wdt", CASES)
def test_irregular_shape_layer_parity(T, H, E, K, I, skew, sent, wdt):
    print(f"shape T={T} H={H} E={E} K={K} I={I} skew={skew} sent={sent} {wdt}", flush=True)
    x, idx, w, w1, w2, dout = _inputs(T, H, E, K, I, T * 31 + E, skew, sent, wdt)
    out_ref, cache = O.experts_forward(x, idx, w, w1, w2)
    dx_ref, dw_ref, dw1_ref, dw2_ref, _ = O.experts_backward(cache, x, w, w1, w2, dout)
    xs, ws, w1s, w2s = (t.to(DEV).requires_grad_(True) for t in (x, w, w1, w2))
    out = experts_forward(xs, idx.to(DEV), ws, w1s, w2s)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    assert _rel(out, out_ref) < TOL
    assert _rel(xs.grad, dx_ref) < TOL
    assert _rel(ws.grad, dw_ref) < TOL
    assert _rel(w1s.grad, dw1_ref) < TOL
    assert _rel(w2s.grad, dw2_ref) < TOL
    used = set(idx[idx < E].reshape(-1).tolist())
    for e in range(E):
        if e not in used:
            assert not w1s.grad[e].any() and not w2s.grad[e].any()


@pytest.mark.parametrize("T,H,E,K,I,skew,sent,wdt", CASES)
def test_irregular_shape_router_parity(T, H, E, K, I, skew, sent, wdt):
    g = torch.Generator().manual_seed(T + 17 * E)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    logits = F.linear(x, wr)
    _, _, idx = ops.router_softmax_topk(logits, K, True)
    _, _, i_ref = O.softmax_router(logits.cpu(), K)
    assert torch.equal(idx.cpu(), i_ref)
    bias = ((torch.rand(E, generator=g) * 2 - 1) * 0.5).to(DEV)
    scores = torch.sigmoid(logits)  # bf16 scores: the selection needs no sigmoid of its own
    w, idx = ops.router_sigmoid_topk_scores(scores, bias, K, True, None, None, None, wdt)
    w_ref, i_ref = O.sigmoid_router_from_scores(scores.cpu(), bias.cpu(), K, True, None, None,
                                                None, wdt)
    assert torch.equal(idx.cpu(), i_ref) and torch.equal(w.cpu(), w_ref)
