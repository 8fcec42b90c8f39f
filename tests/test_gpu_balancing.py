"""GPU parity of the routing consumers (moe_amd.balancing, balance.hip)
against the CPU oracle on the same inputs: selection counts bit-exact (inputs
without exact ties), sums, losses and statistics within 1e-6 relative (fp32
data, fp64 sums in a different order), gradients within 1e-5 of the largest
(fp32 kernels vs the fp64 autograd of the oracle), bias updates bit-exact."""
from __future__ import annotations

import math

import pytest
import torch

from moe_amd import balancing as Bal
from moe_amd.router import MI355XDeepSeekRouter
from oracle import balancing_oracle as B
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _probs(T, E, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.softmax(torch.randn(T, E, generator=g) * 2, dim=-1).to(dtype)


def _close(a, b, rel=1e-6):
    return abs(a - b) <= rel * max(abs(b), 1e-30)


@pytest.mark.parametrize("T,E,K,dtype,weighted", [
    (4096, 128, 8, torch.float32, False),
    (1000, 100, 3, torch.float32, True),     # E not a multiple of 64, mask weights
    (512, 1792, 8, torch.float32, False),    # retrofit bank width
    (777, 64, 1, torch.bfloat16, False),
    (300, 16, 16, torch.float32, False),     # K == E: no margin
])
def test_topk_stats_parity(T, E, K, dtype, weighted):
    print(f"topk_stats T={T} E={E} K={K} {dtype} weighted={weighted}", flush=True)
    p = _probs(T, E, T + E, dtype)
    w = (torch.rand(T, generator=torch.Generator().manual_seed(1)) > 0.3).float() if weighted else None
    counts, sums, margin = Bal.topk_stats(p.to(DEV), K, None if w is None else w.to(DEV))
    torch.cuda.synchronize()
    pd = p.double()
    _, idx = O.rank_topk(pd, K)
    ww = torch.ones(T, dtype=torch.float64) if w is None else w.double()
    ref_c = torch.zeros(E, dtype=torch.float64).index_add_(0, idx.reshape(-1),
                                                           ww.repeat_interleave(K))
    assert torch.equal(counts.cpu(), ref_c)
    ref_s = (pd * ww[:, None]).sum(0)
    assert ((sums.cpu() - ref_s).abs() <= 1e-5 * ref_s.abs().max()).all()
    if K < E:
        srt = pd.sort(dim=-1, descending=True).values
        m = srt[:, K - 1] - srt[:, K]
        assert _close(margin[0].item(), m.sum().item(), 1e-5)
        assert margin[1].item() == pytest.approx(m.min().item(), abs=1e-7)


@pytest.mark.parametrize("masked", [False, True])
def test_switch_loss_and_gradient(masked):
    bsz, S, E, K, L = 2, 512, 64, 4, 3
    print(f"switch loss masked={masked}", flush=True)
    layers = [_probs(bsz * S, E, 10 + i) for i in range(L)]
    mask = None
    if masked:
        mask = torch.ones(bsz, S)
        mask[0, 400:] = 0
        mask[1, :50] = 0
    ref_in = [x.double().requires_grad_(True) for x in layers]
    ref = B.switch_aux_loss(tuple(ref_in), E, K, attention_mask=mask)
    ref_g = torch.autograd.grad(ref, ref_in)
    gin = [x.to(DEV).requires_grad_(True) for x in layers]
    loss = Bal.load_balancing_loss_func(tuple(gin), E, K,
                                        attention_mask=None if mask is None else mask.to(DEV))
    loss.backward()
    torch.cuda.synchronize()
    assert _close(loss.item(), ref.item())
    for gi, rg in zip(gin, ref_g):
        assert (gi.grad.double().cpu() - rg).abs().max() <= 1e-5 * rg.abs().max()
    assert Bal.load_balancing_loss_func(None, E, K) == 0
    assert Bal.load_balancing_loss_func([gin[0]], E, K) == 0   # not a tuple


@pytest.mark.parametrize("bsz,S,E,K,given,dtype", [
    (4, 128, 64, 8, False, torch.float32),
    (2, 300, 100, 4, True, torch.float32),
    (1, 256, 256, 8, False, torch.bfloat16),
])
def test_seq_loss_and_gradient(bsz, S, E, K, given, dtype):
    print(f"seq loss B={bsz} S={S} E={E} K={K} given={given} {dtype}", flush=True)
    g = torch.Generator().manual_seed(S + E)
    layers = [torch.sigmoid(torch.randn(bsz * S, E, generator=g)).to(dtype) for _ in range(2)]
    sel = None
    if given:
        sel = tuple(torch.randint(0, E, (bsz * S, K), generator=g) for _ in layers)
    ref_in = [x.double().requires_grad_(True) for x in layers]
    ref = B.seq_aux_loss(tuple(ref_in), E, K, bsz, sel)
    ref_g = torch.autograd.grad(ref, ref_in)
    gin = [x.to(DEV).requires_grad_(True) for x in layers]
    loss = Bal.seq_load_balancing_loss_func(
        tuple(gin), E, K, batch_size=bsz,
        selected_experts=None if sel is None else tuple(s.to(DEV) for s in sel))
    loss.backward()
    torch.cuda.synchronize()
    tol = 1e-6 if dtype == torch.float32 else 1e-5
    assert _close(loss.item(), ref.item(), tol)
    for gi, rg in zip(gin, ref_g):
        lim = (2e-2 if dtype == torch.bfloat16 else 1e-5) * rg.abs().max()
        assert (gi.grad.double().cpu() - rg).abs().max() <= lim


def test_routing_stats_and_counts():
    L, T, E, K = 3, 2048, 64, 4
    layers = [_probs(T, E, 30 + i) for i in range(L)]
    ref = B.routing_stats(layers, K, is_global=True)
    got = Bal.compute_routing_stats([x.to(DEV) for x in layers], K, is_global=True)
    assert set(got) == set(ref)
    for k, v in ref.items():
        if isinstance(v, list):
            assert len(got[k]) == len(v)
            assert all(abs(a - b) <= 1e-9 + 1e-6 * abs(b) for a, b in zip(got[k], v)), k
        elif isinstance(v, int):
            assert got[k] == v, k
        else:
            assert abs(got[k] - v) <= 1e-6 * max(abs(v), 1e-3), (k, got[k], v)
    acc = Bal.accumulate_expert_counts([x.to(DEV) for x in layers], K)
    acc = Bal.accumulate_expert_counts([x.to(DEV) for x in layers], K, acc)
    for i, x in enumerate(layers):
        assert torch.equal(acc[i].cpu(), 2 * B._counts(x.double(), K).float())
    tab = Bal.expert_counts_to_tables(acc, is_global=True)
    assert len(tab["_table/global_pool_expert_tokens"]) == E


class _Model(torch.nn.Module):
    def __init__(self, L, E, H=64):
        super().__init__()
        from transformers import Qwen3MoeConfig
        cfg = Qwen3MoeConfig(hidden_size=H, num_experts=E, num_experts_per_tok=2,
                             num_hidden_layers=L, num_attention_heads=4, num_key_value_heads=2,
                             moe_intermediate_size=32, intermediate_size=128, vocab_size=128)
        self.routers = torch.nn.ModuleList(MI355XDeepSeekRouter(cfg) for _ in range(L))


@pytest.mark.parametrize("is_global,alpha", [(False, 0.0), (True, 0.0), (True, 0.3)])
def test_update_expert_biases(is_global, alpha):
    print(f"bias update global={is_global} alpha={alpha}", flush=True)
    L, E = 4, 96
    model = _Model(L, E).to(DEV)
    g = torch.Generator().manual_seed(L + E)
    counts = [torch.randint(0, 300, (E,), generator=g).float() for _ in range(L)]
    biases = [torch.randn(E, generator=g) * 0.1 for _ in range(L)]
    for r, c, b in zip(model.routers, counts, biases):
        r.local_tokens_per_expert.copy_(c)
        r.expert_bias.copy_(b)
    want, want_st = B.update_expert_biases(counts, biases, 1e-3, is_global, alpha)
    st = Bal.update_expert_biases(model, 1e-3, None, is_global=is_global, alpha=alpha)
    torch.cuda.synchronize()
    for r, w in zip(model.routers, want):
        assert torch.equal(r.expert_bias.cpu(), w)
        assert not r.local_tokens_per_expert.any()
    for k, v in want_st.items():
        assert abs(st[k] - v) <= 1e-12 + 1e-9 * abs(v), k
    assert Bal.update_expert_biases(torch.nn.Linear(2, 2).to(DEV), 1e-3) == {}
