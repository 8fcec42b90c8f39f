"""The drop-in boundary: the C ABI surface and the transformers plug-in.

CPU tests: the library exports every symbol include/moe_amd.h declares, the
ctypes prototypes match the header's parameter counts, the "mi355x" key
registers in transformers' ExpertsInterface, install() swaps routers in place
without changing state_dict keys, and CPU tensors are refused (no fallback).
GPU tests: a tiny Qwen3MoeForCausalLM runs fwd+bwd through the HIP path, its
MoE blocks match the oracle, and a bank shared by two routers (the reference's
global bank) accumulates both calls' weight gradients.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch
from torch import nn

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "moe_amd.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|size_t|const char\*)\s+(moe_amd_\w+)\(([^)]*)\)", text):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else len(args.split(","))
    return out


def test_header_declares_entry_points():
    decl = _declared()
    assert len(decl) >= 18
    assert "moe_amd_permute" in decl and "moe_amd_gemm_gate_up_swiglu" in decl


def test_library_exports_every_declared_symbol(built_lib):
    lib = ctypes.CDLL(str(built_lib))
    for name in _declared():
        assert hasattr(lib, name), f"{name} not exported"


def test_ctypes_prototypes_match_header():
    from moe_amd import _lib
    decl = _declared()
    assert set(decl) == set(_lib.SIGNATURES)
    for name, n in decl.items():
        assert len(_lib.SIGNATURES[name][1]) == n, name


def test_abi_version_and_error_text(built_lib):
    from moe_amd import _lib
    lib = _lib.load()
    assert lib.moe_amd_abi_version() == 1
    # Argument validation runs on the host: no GPU needed to see the error path.
    rc = lib.moe_amd_permute(None, 10, 0, None, 0, None, None, None, None, None, 0, None)
    assert rc == -1
    assert "E=0" in _lib.last_error()
    rc = lib.moe_amd_gemm_down(None, None, None, None, 16, 4, 100, 64, 1, None, None)
    assert rc == -1 and "multiples of 64" in _lib.last_error()
    # fp32 is a supported GEMM dtype (its own kernels): the null pointers are the error
    rc = lib.moe_amd_gemm_down(None, None, None, None, 16, 4, 128, 64, 0, None, None)
    assert rc == -1 and "null pointer" in _lib.last_error() and "fp32" in _lib.last_error()
    rc = lib.moe_amd_gemm_down(None, None, None, None, 16, 4, 128, 64, 7, None, None)
    assert rc == -2 and "neither bf16 nor fp32" in _lib.last_error()
    # the fused combine + GEMM-2 backward is bf16 only
    rc = lib.moe_amd_gemm_down_backward_dx_fused(None, None, 2, None, None, None, None, None, 0,
                                                 8, 16, 4, 128, 64, 0, None, None, None, None)
    assert rc == -6 and "bf16 only" in _lib.last_error()


def _tiny_model():
    from transformers import Qwen3MoeConfig, Qwen3MoeForCausalLM
    cfg = Qwen3MoeConfig(vocab_size=256, hidden_size=128, intermediate_size=256,
                         moe_intermediate_size=64, num_hidden_layers=2, num_attention_heads=2,
                         num_key_value_heads=1, head_dim=64, num_experts=8,
                         num_experts_per_tok=2, norm_topk_prob=True, decoder_sparse_step=1,
                         max_position_embeddings=128)
    torch.manual_seed(0)
    m = Qwen3MoeForCausalLM(cfg)
    with torch.no_grad():
        for n, p in m.named_parameters():
            if "experts" in n or "gate.weight" in n:
                p.normal_(0, 0.02)
    return m


def test_register_and_install_swap_in_place():
    from transformers.integrations.moe import ALL_EXPERTS_FUNCTIONS
    from moe_amd import hf
    from moe_amd.router import MI355XTopKRouter
    m = _tiny_model()
    keys = list(m.state_dict().keys())
    w_before = m.model.layers[0].mlp.gate.weight
    hf.install(m)
    assert "mi355x" in ALL_EXPERTS_FUNCTIONS
    assert m.config._experts_implementation == "mi355x"
    assert m.model.layers[0].mlp.experts.config._experts_implementation == "mi355x"
    assert isinstance(m.model.layers[1].mlp.gate, MI355XTopKRouter)
    assert m.model.layers[0].mlp.gate.weight is w_before
    assert list(m.state_dict().keys()) == keys
    with pytest.raises(RuntimeError, match="GPU only"):
        m(torch.randint(0, 256, (1, 8)))


def test_deepseek_router_swap_keeps_buffers():
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeTopKRouter
    from moe_amd import hf
    from moe_amd.router import MI355XDeepSeekRouter

    class BiasRouter(Qwen3MoeTopKRouter):  # stands in for the reference's DeepSeekRouter
        def __init__(self, config):
            super().__init__(config)
            self.scaling_factor = 2.5
            self.num_groups = None
            self.group_topk = None
            self.register_buffer("expert_bias", torch.randn(config.num_experts))
            self.register_buffer("local_tokens_per_expert", torch.zeros(config.num_experts),
                                 persistent=False)

    cfg = SimpleNamespace(num_experts_per_tok=4, num_experts=16, norm_topk_prob=True,
                          hidden_size=64)
    holder = nn.Module()
    holder.gate = BiasRouter(cfg)
    sd = holder.state_dict()
    assert hf.swap_routers(holder) == 1
    assert isinstance(holder.gate, MI355XDeepSeekRouter)
    assert holder.gate.scaling_factor == 2.5
    new_sd = holder.state_dict()
    assert set(new_sd) == set(sd) == {"gate.weight", "gate.expert_bias"}
    assert torch.equal(new_sd["gate.expert_bias"], sd["gate.expert_bias"])


def test_unsupported_expert_variants_raise():
    from moe_amd.experts import mi355x_experts_forward
    fake = SimpleNamespace(has_gate=True, has_bias=True, is_transposed=False)
    with pytest.raises(NotImplementedError):
        mi355x_experts_forward(fake, None, None, None)


# ------------------------------------------------------------------ GPU

@pytest.mark.gpu
def test_tiny_hf_model_runs_on_hip_path_and_matches_oracle():
    from oracle import moe_oracle as O
    from moe_amd import hf
    m = _tiny_model().to("cuda", torch.bfloat16)
    hf.install(m)
    captured = []
    blk = m.model.layers[1].mlp
    blk.register_forward_hook(lambda mod, inp, out: captured.append((inp[0].detach(),
                                                                     out.detach())))
    ids = torch.randint(0, 256, (2, 32), device="cuda")
    out = m(ids, labels=ids, output_router_logits=True)
    assert torch.isfinite(out.loss)
    assert len(out.router_logits) == 2 and out.router_logits[0].shape == (64, 8)
    out.loss.backward()
    assert blk.experts.gate_up_proj.grad is not None and blk.gate.weight.grad is not None
    h, y = captured[0]
    flat = h.reshape(-1, 128)
    logits = torch.nn.functional.linear(flat, blk.gate.weight).cpu()
    _, w, idx = O.softmax_router(logits, 2)
    ref, _ = O.experts_forward(flat.cpu(), idx, w, blk.experts.gate_up_proj.detach().cpu(),
                               blk.experts.down_proj.detach().cpu())
    err = (y.reshape(-1, 128).double().cpu() - ref.double()).abs().max() / ref.abs().max()
    assert err < 2e-2


@pytest.mark.gpu
def test_shared_bank_accumulates_gradients_across_layers():
    """One expert bank used by two routers (GlobalMoEModel's global_experts,
    src/models/global_moe.py:138): its dW is the sum of both calls'."""
    from oracle import moe_oracle as O
    from moe_amd.layer import moe_layer
    g = torch.Generator().manual_seed(5)
    T, H, E, K, I = 512, 256, 32, 4, 128
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    r = [(torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16) for _ in range(2)]
    d = [torch.randn(T, H, generator=g).to(torch.bfloat16) for _ in range(2)]
    w1d = w1.cuda().requires_grad_(True)
    w2d = w2.cuda().requires_grad_(True)
    for layer in range(2):
        out, _, _, _ = moe_layer(x.cuda(), r[layer].cuda(), w1d, w2d, K, gating="torch")
        out.backward(d[layer].cuda())
    torch.cuda.synchronize()
    acc1 = torch.zeros(E, 2 * I, H, dtype=torch.float64)
    acc2 = torch.zeros(E, H, I, dtype=torch.float64)
    for layer in range(2):
        logits = torch.nn.functional.linear(x.cuda(), r[layer].cuda()).cpu()
        _, w, idx = O.softmax_router(logits, K)
        _, cache = O.experts_forward(x, idx, w, w1, w2)
        _, _, dw1, dw2, _ = O.experts_backward(cache, x, w, w1, w2, d[layer])
        acc1 += dw1.double()
        acc2 += dw2.double()
    e1 = (w1d.grad.double().cpu() - acc1).abs().max() / acc1.abs().max()
    e2 = (w2d.grad.double().cpu() - acc2).abs().max() / acc2.abs().max()
    assert e1 < 2e-2 and e2 < 2e-2


@pytest.mark.gpu
@pytest.mark.parametrize("main_grad", [False, True])
def test_global_bank_dispatches_through_experts_interface(main_grad):
    """The global shared bank as the reference builds it (src/models/
    global_moe.py:45-66, :130-151), from transformers classes only: one
    Qwen3MoeExperts owned by a Qwen3MoeModel and called by two router-only
    blocks (a Qwen3MoeTopKRouter each).  After hf.install() both calls
    dispatch through the "mi355x" ExpertsInterface key (counted), the gates
    are the HIP routers, and the bank's dW is the oracle's sum over both
    calls -- in .grad, or, with main_grad buffers on the bank's two
    parameters, accumulated in place into them with .grad left None."""
    import copy
    from unittest import mock
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import (Qwen3MoeExperts, Qwen3MoeModel,
                                                                  Qwen3MoeTopKRouter)
    from oracle import moe_oracle as O
    from moe_amd import experts as experts_mod
    from moe_amd import hf
    from moe_amd.router import MI355XTopKRouter

    cfg = Qwen3MoeConfig(vocab_size=64, hidden_size=256, intermediate_size=256,
                         moe_intermediate_size=128, num_hidden_layers=2, num_attention_heads=2,
                         num_key_value_heads=1, head_dim=64, num_experts=32,
                         num_experts_per_tok=4, norm_topk_prob=True,
                         max_position_embeddings=64)

    class RouterOnlyBlock(nn.Module):  # global_moe.py:45-66, restated
        def __init__(self, config):
            super().__init__()
            self.gate = Qwen3MoeTopKRouter(config)

        def forward(self, hidden_states, global_experts):
            B, T, H = hidden_states.shape
            flat = hidden_states.view(-1, H)
            _, routing_weights, selected_experts = self.gate(flat)
            return global_experts(flat, selected_experts, routing_weights).reshape(B, T, H)

    dense = copy.deepcopy(cfg)
    dense.mlp_only_layers = list(range(cfg.num_hidden_layers))
    torch.manual_seed(0)
    model = Qwen3MoeModel(dense)
    model.config = cfg
    model.global_experts = Qwen3MoeExperts(cfg)  # one bank, registered once (:138)
    for layer in model.layers:
        layer.mlp = RouterOnlyBlock(cfg)
    with torch.no_grad():
        for n, p in model.named_parameters():
            if "global_experts" in n or "gate.weight" in n:
                p.normal_(0, 0.02)
    model = model.to("cuda", torch.bfloat16)
    hf.install(model)
    bank = model.global_experts
    assert bank.config._experts_implementation == "mi355x"
    assert all(isinstance(layer.mlp.gate, MI355XTopKRouter) for layer in model.layers)
    if main_grad:
        for p in (bank.gate_up_proj, bank.down_proj):
            p.main_grad = torch.zeros_like(p)

    g = torch.Generator().manual_seed(3)
    B, T, H, K = 2, 64, cfg.hidden_size, cfg.num_experts_per_tok
    hs = [torch.randn(B, T, H, generator=g).to(torch.bfloat16) for _ in range(2)]
    ds = [torch.randn(B, T, H, generator=g).to(torch.bfloat16) for _ in range(2)]
    calls = []
    real = experts_mod.experts_forward

    def counting(*a, **k):
        calls.append(a[0].shape)
        return real(*a, **k)

    with mock.patch.object(experts_mod, "experts_forward", counting):
        loss = 0
        for layer, h, d in zip(model.layers, hs, ds):
            out = layer.mlp(h.cuda(), bank)
            loss = loss + (out.float() * d.cuda().float()).sum()
        loss.backward()
    torch.cuda.synchronize()
    assert len(calls) == 2, "each router-only block's call must dispatch through mi355x"
    w1c = bank.gate_up_proj.detach().cpu()
    w2c = bank.down_proj.detach().cpu()
    acc1 = torch.zeros(w1c.shape, dtype=torch.float64)
    acc2 = torch.zeros(w2c.shape, dtype=torch.float64)
    for layer, h, d in zip(model.layers, hs, ds):
        flat = h.reshape(-1, H)
        logits = torch.nn.functional.linear(flat.cuda(), layer.mlp.gate.weight).cpu()
        _, w, idx = O.softmax_router(logits, K)
        _, cache = O.experts_forward(flat, idx, w, w1c, w2c)
        _, _, dw1, dw2, _ = O.experts_backward(cache, flat, w, w1c, w2c, d.reshape(-1, H))
        acc1 += dw1.double()
        acc2 += dw2.double()
    if main_grad:
        assert bank.gate_up_proj.grad is None and bank.down_proj.grad is None
        g1, g2 = bank.gate_up_proj.main_grad, bank.down_proj.main_grad
    else:
        g1, g2 = bank.gate_up_proj.grad, bank.down_proj.grad
    e1 = (g1.double().cpu() - acc1).abs().max() / acc1.abs().max()
    e2 = (g2.double().cpu() - acc2).abs().max() / acc2.abs().max()
    print(f"global bank dW over two calls (main_grad={main_grad}): {e1:.2e} {e2:.2e}", flush=True)
    assert e1 < 2e-2 and e2 < 2e-2


@pytest.mark.gpu
@pytest.mark.parametrize("router", ["softmax", "deepseek"])
def test_tiny_hf_model_under_bf16_autocast(router):
    """The reference's training precision: fp32 parameters (the model is
    built from its config and never cast, train.py:193-235) and the forward
    under bf16 autocast (Accelerator(mixed_precision="bf16"), train.py:395-400).
    The gating linear then yields bf16 logits; the routing must be the
    reference's on them and the experts run in the weights' fp32, as
    transformers' grouped_mm does (it casts the input to the weight dtype).
    The second block's output is checked against the oracle at the fp32
    bound, and every parameter gradient is fp32 and finite."""
    import torch.nn.functional as F

    from oracle import moe_oracle as O
    from moe_amd import hf
    from moe_amd.router import MI355XDeepSeekRouter
    print(f"tiny HF model under bf16 autocast, {router} router", flush=True)
    m = _tiny_model().to("cuda")
    cfg = m.config
    if router == "deepseek":
        g = torch.Generator().manual_seed(3)
        for layer in m.model.layers:
            new = MI355XDeepSeekRouter(cfg).to("cuda")
            new.weight = layer.mlp.gate.weight
            new.expert_bias.copy_((torch.rand(cfg.num_experts, generator=g) - 0.5).to("cuda"))
            layer.mlp.gate = new
    hf.install(m)
    blk = m.model.layers[1].mlp
    captured = []
    blk.register_forward_hook(lambda mod, inp, out: captured.append((inp[0].detach(),
                                                                     out.detach())))
    ids = torch.randint(0, 256, (2, 32), device="cuda")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = m(ids, labels=ids)
    out.loss.backward()
    assert torch.isfinite(out.loss)
    for p in (blk.experts.gate_up_proj, blk.experts.down_proj, blk.gate.weight):
        assert p.grad is not None and p.grad.dtype == torch.float32
        assert torch.isfinite(p.grad).all()
    h, y = captured[0]
    flat = h.reshape(-1, cfg.hidden_size)
    K = cfg.num_experts_per_tok
    with torch.autocast("cuda", dtype=torch.bfloat16):
        if router == "softmax":
            logits = F.linear(flat, blk.gate.weight)
        else:
            logits = F.linear(flat.float(), blk.gate.weight.float())
    assert logits.dtype == torch.bfloat16
    if router == "softmax":
        _, w, idx = O.softmax_router(logits.cpu(), K)
    else:
        w, idx = O.sigmoid_router_from_scores(torch.sigmoid(logits).cpu(),
                                              blk.gate.expert_bias.cpu(), K, True,
                                              weights_dtype=flat.dtype)
    # the experts compute in the weights' dtype (fp32), their input cast to it
    ref, _ = O.experts_forward(flat.float().cpu(), idx, w, blk.experts.gate_up_proj.detach().cpu(),
                               blk.experts.down_proj.detach().cpu())
    assert y.dtype == flat.dtype
    err = (y.reshape(-1, cfg.hidden_size).double().cpu() - ref.double()).abs().max() \
        / ref.abs().max()
    assert err < 1e-5, float(err)
