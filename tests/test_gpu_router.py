"""GPU parity of the router kernels against the CPU oracle.

Routing indices are compared bit-exactly; probabilities / weights / gradients
within fp32 tolerance (rtol 1e-5).  Logits come from one torch F.linear on
the GPU and are handed to both sides, so kernel and oracle see the same bits.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from moe_amd import ops
from moe_amd.router import sigmoid_topk, softmax_topk
from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs().max() / b.abs().max().clamp_min(1e-30)).item()


@pytest.mark.parametrize("T,H,E,K,dtype", [
    (2048, 1024, 16, 4, torch.float32),      # XS standard shape
    (4096, 1024, 128, 4, torch.bfloat16),    # XS global bank (token sample)
    (8192, 2048, 128, 8, torch.bfloat16),    # L / M shape (token sample)
    (512, 256, 1792, 8, torch.bfloat16),     # retrofit expert count
    (333, 128, 60, 6, torch.bfloat16),       # ragged sizes
    (1000, 256, 256, 12, torch.bfloat16),    # 16 lanes per token, K > 8
    (777, 128, 200, 8, torch.bfloat16),      # 16 lanes per token, partly empty lanes
    (100, 64, 1, 1, torch.bfloat16),         # one expert
    (257, 64, 8, 1, torch.float32),          # top-1
    (64, 64, 4, 4, torch.bfloat16),          # K = E
])
def test_softmax_router_parity(T, H, E, K, dtype):
    print(f"softmax router T={T} H={H} E={E} K={K} {dtype}", flush=True)
    g = torch.Generator().manual_seed(T + E)
    x = torch.randn(T, H, generator=g).to(dtype).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(dtype).to(DEV)
    logits = F.linear(x, wr)
    tpe = torch.zeros(E, device=DEV)
    probs, w, idx = ops.router_softmax_topk(logits, K, True, tokens_per_expert=tpe)
    torch.cuda.synchronize()
    p_ref, w_ref, i_ref = O.softmax_router(logits.cpu(), K)
    assert torch.equal(idx.cpu(), i_ref), "routing indices differ"
    assert torch.allclose(probs.cpu(), p_ref, rtol=1e-5, atol=1e-7)
    assert torch.allclose(w.cpu(), w_ref, rtol=1e-5, atol=1e-7)
    counts = torch.bincount(i_ref.reshape(-1), minlength=E).float()
    assert torch.equal(tpe.cpu(), counts)


def test_softmax_router_ties_and_offset():
    """Quantised logits make exact ties common at the selection boundary."""
    g = torch.Generator().manual_seed(11)
    T, E, K = 4096, 128, 8
    logits = (torch.randint(-6, 7, (T, E), generator=g).float() / 4).to(torch.bfloat16).to(DEV)
    off = (2.0 * (torch.randperm(E, generator=g).float() + 1).pow(-1.1)).to(DEV)
    for offset in (None, off):
        probs, w, idx = ops.router_softmax_topk(logits, K, True, logit_offset=offset)
        p_ref, w_ref, i_ref = O.softmax_router(logits.cpu(), K, True,
                                               None if offset is None else offset.cpu())
        assert torch.equal(idx.cpu(), i_ref)
        assert torch.allclose(w.cpu(), w_ref, rtol=1e-5, atol=1e-7)
    # Hand-derived: all-equal logits select experts 0..K-1 with weight 1/K.
    flat = torch.zeros(3, E, dtype=torch.bfloat16, device=DEV)
    _, w0, i0 = ops.router_softmax_topk(flat, K, True)
    assert i0.cpu().tolist() == [list(range(K))] * 3
    assert torch.allclose(w0.cpu(), torch.full((3, K), 1.0 / K))


def test_torch_topk_tie_order_probe():
    """Records how torch.topk on this device orders exact ties (informational:
    the reference calls torch.topk; the kernel and oracle use lower-id-first)."""
    v = torch.zeros(4, 128, device=DEV)
    v[:, 5] = 1.0
    _, i = torch.topk(v, 8, dim=-1)
    print("torch.topk tie order on device:", i[0].tolist(), flush=True)
    assert i[0, 0].item() == 5


@pytest.mark.parametrize("T,H,E,K,groups,gtk,sf,wdt", [
    (2048, 2048, 1792, 8, None, None, None, torch.bfloat16),   # retrofit router
    (1024, 256, 128, 8, 8, 4, 2.5, torch.float32),             # DeepSeek grouped YAMLs
    (513, 128, 64, 6, None, None, 2.5, torch.float32),
    (2000, 512, 128, 8, None, None, None, torch.bfloat16),   # DeepSeek YAMLs' E, flat top-k
    (999, 256, 100, 4, None, None, None, torch.float32),      # lanes partly empty
    (600, 256, 256, 12, None, None, 1.5, torch.bfloat16),     # 16 lanes per token
    (700, 128, 300, 16, None, None, None, torch.float32),     # 4 waves per token, 2 slots, K=16
    (333, 128, 520, 8, None, None, 2.0, torch.bfloat16),      # 4 waves per token, ragged slots
    (100, 64, 4000, 8, None, None, None, torch.float32),      # 4 waves per token, 16 slots
    (300, 128, 1792, 20, None, None, None, torch.float32),    # K > 16: one wave per token
    (256, 128, 1792, 8, 8, 4, None, torch.float32),           # grouped at the retrofit E
])
def test_sigmoid_router_parity(T, H, E, K, groups, gtk, sf, wdt):
    print(f"sigmoid router T={T} E={E} K={K} groups={groups}", flush=True)
    g = torch.Generator().manual_seed(T + E + 1)
    x = torch.randn(T, H, generator=g).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(DEV)
    bias = ((torch.rand(E, generator=g) * 2 - 1) * 0.5).to(DEV)
    logits = F.linear(x.float(), wr.float())
    tpe = torch.zeros(E, device=DEV)
    scores, w, idx = ops.router_sigmoid_topk(logits, bias, K, True, sf, groups, gtk, wdt, tpe)
    torch.cuda.synchronize()
    # The scores are torch.sigmoid's on this device bit for bit (the
    # reference's call, router.py:112); selection and weights are then
    # exact against the oracle on those scores.
    s_dev = torch.sigmoid(logits)
    assert torch.equal(scores, s_dev), "scores differ from torch.sigmoid on the device"
    sc = s_dev.cpu()
    assert torch.allclose(sc, torch.sigmoid(logits.cpu()), rtol=2e-6, atol=1e-7)
    w_ref, i_ref = O.sigmoid_router_from_scores(sc, bias.cpu(), K, True, sf, groups, gtk, wdt)
    assert torch.equal(idx.cpu(), i_ref), "selection differs from the oracle's"
    assert torch.allclose(w.cpu().float(), w_ref.float(), rtol=1e-5 if wdt == torch.float32
                          else 8e-3, atol=1e-7)
    counts = torch.bincount(idx.cpu().reshape(-1), minlength=E).float()
    assert torch.equal(tpe.cpu(), counts)
    if groups is not None:
        assert all(len(set((r // (E // groups)).tolist())) <= gtk for r in idx.cpu())
    if sf:  # bf16 weights: K roundings of up to half an ulp each
        assert torch.allclose(w.float().sum(-1).cpu(), torch.full((T,), float(sf)),
                              atol=1e-4 if wdt == torch.float32 else K * float(sf) * 2.0 ** -9)


def test_sigmoid_router_no_nan_at_zero_scores():
    logits = torch.full((8, 64), -6400.0, device=DEV)
    _, w, _ = ops.router_sigmoid_topk(logits, None, 4, True, None, None, None, torch.float32)
    assert torch.isfinite(w).all()


@pytest.mark.parametrize("renorm", [True, False])
@pytest.mark.parametrize("E,K,with_dp", [(128, 8, True), (128, 8, False), (64, 6, True),
                                         (256, 12, False), (60, 6, True)])
def test_softmax_router_backward_parity(renorm, E, K, with_dp):
    print(f"softmax router backward E={E} K={K} renorm={renorm} d_probs={with_dp}", flush=True)
    g = torch.Generator().manual_seed(21 + E + K)
    T = 2048 + 3
    logits = (torch.randn(T, E, generator=g)).to(torch.bfloat16).to(DEV).requires_grad_(True)
    probs, w, idx = softmax_topk(logits, K, renorm, None)
    dw = torch.randn(T, K, generator=g).to(DEV)
    dp = torch.randn(T, E, generator=g).to(DEV) * 0.1
    if not with_dp:
        dp = torch.zeros_like(dp)
    loss = (w * dw).sum() + ((probs * dp).sum() if with_dp else 0)
    (gl,) = torch.autograd.grad(loss, logits)
    ref = O.softmax_router_backward(probs.detach().cpu(), idx.cpu(), dw.cpu(), dp.cpu(), renorm,
                                    torch.float32)
    assert gl.dtype == torch.bfloat16
    assert _rel(gl.float(), ref) < 1e-2  # bf16 output rounding


@pytest.mark.parametrize("E,K,wdt", [(256, 8, torch.float32), (128, 8, torch.bfloat16),
                                     (100, 4, torch.float32), (1792, 8, torch.bfloat16)])
def test_sigmoid_router_backward_parity(E, K, wdt):
    print(f"sigmoid router backward E={E} K={K} {wdt}", flush=True)
    g = torch.Generator().manual_seed(22 + E)
    T = 1024 + 5
    logits = torch.randn(T, E, generator=g).to(DEV).requires_grad_(True)
    bias = (torch.rand(E, generator=g) - 0.5).to(DEV)
    scores, w, idx = sigmoid_topk(logits, bias, K, True, 2.5, None, None, wdt, None)
    dw = torch.randn(T, K, generator=g).to(DEV)
    ds = torch.randn(T, E, generator=g).to(DEV) * 0.1
    (gl,) = torch.autograd.grad((w.float() * dw).sum() + (scores * ds).sum(), logits)
    ref = O.sigmoid_router_backward(scores.detach().cpu(), idx.cpu(), dw.to(wdt).float().cpu(),
                                    ds.cpu(), True, 2.5)
    assert torch.allclose(gl.cpu(), ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("T,E,K,groups,gtk,sf,renorm,wdt", [
    (2048, 128, 8, None, None, None, True, torch.bfloat16),   # group kernel, 16-byte rows
    (777, 100, 6, None, None, 2.5, True, torch.float32),      # group kernel, element rows
    (512, 1792, 8, None, None, None, True, torch.bfloat16),   # four waves per token
    (300, 256, 8, 8, 4, None, True, torch.float32),           # group-limited, wave per token
    (400, 2304, 20, None, None, None, False, torch.bfloat16),  # K > 16: wave per token
])
def test_sigmoid_router_bf16_scores_parity(T, E, K, groups, gtk, sf, renorm, wdt):
    """The DeepSeek router from bf16 scores (the reference under bf16
    autocast): index and weights bit-identical to the oracle's evaluation of
    router.py:114-140 on the same scores, counts exact."""
    print(f"sigmoid router from bf16 scores T={T} E={E} K={K} groups={groups}", flush=True)
    g = torch.Generator().manual_seed(T + E + 7)
    logits = (torch.randn(T, E, generator=g) * 2).to(torch.bfloat16).to(DEV)
    bias = ((torch.rand(E, generator=g) * 2 - 1) * 0.5).to(DEV)
    scores = torch.sigmoid(logits)
    tpe = torch.zeros(E, device=DEV)
    w, idx = ops.router_sigmoid_topk_scores(scores, bias, K, renorm, sf, groups, gtk, wdt, tpe)
    torch.cuda.synchronize()
    w_ref, i_ref = O.sigmoid_router_from_scores(scores.cpu(), bias.cpu(), K, renorm, sf, groups,
                                                gtk, wdt)
    assert torch.equal(idx.cpu(), i_ref)
    assert torch.equal(w.cpu(), w_ref)
    assert torch.equal(tpe.cpu(), torch.bincount(i_ref.reshape(-1), minlength=E).float())


def test_sigmoid_layer_op_takes_bf16_logits():
    """moe_amd::sigmoid_topk on bf16 logits: bf16 scores as torch.sigmoid
    gives them, the from-scores selection, and a backward through the
    sigmoid in the logits' dtype."""
    g = torch.Generator().manual_seed(5)
    T, E, K = 1024, 128, 8
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16).to(DEV).requires_grad_(True)
    bias = (torch.rand(E, generator=g) - 0.5).to(DEV)
    scores, w, idx = sigmoid_topk(logits, bias, K, True, None, None, None, torch.bfloat16, None)
    assert scores.dtype == torch.bfloat16 and torch.equal(scores, torch.sigmoid(logits))
    w_ref, i_ref = O.sigmoid_router_from_scores(scores.detach().cpu(), bias.cpu(), K, True,
                                                weights_dtype=torch.bfloat16)
    assert torch.equal(idx.cpu(), i_ref) and torch.equal(w.cpu(), w_ref)
    dw = torch.randn(T, K, generator=g).to(DEV)
    (gl,) = torch.autograd.grad((w.float() * dw).sum(), logits)
    ref = O.sigmoid_router_backward(scores.detach().float().cpu(), idx.cpu(),
                                    dw.to(torch.bfloat16).float().cpu(), None, True, None)
    assert gl.dtype == torch.bfloat16
    assert _rel(gl.float(), ref) < 1e-2  # bf16 rounding of the gradient


@pytest.mark.parametrize("T,H,E", [
    (65536, 2048, 128),   # L router GEMM
    (4096, 2048, 1792),   # retrofit expert count (token sample)
    (2048, 1024, 16),     # XS expert count
    (1001, 128, 8),       # ragged T, one column tile mostly empty
    (256, 64, 264),       # E just past one 256-column tile
    (3000, 512, 200),     # transposed form, 256-expert row tile, ragged T
    (700, 256, 256),      # transposed form, full 256-expert row tile
    (77, 1024, 64),       # transposed form, fewer tokens than one column tile
    (1500, 320, 96),      # transposed form, 5 k-stages: every rotated k start, wrapping
])
def test_router_linear_parity(T, H, E):
    """The MFMA gating linear against fp32 torch on the same bf16 inputs: the
    fp32 output within 1e-5 of max|logit| (products of bf16 values are exact in
    fp32, only the summation order differs), the bf16 output within one bf16
    rounding of the fp32 result."""
    print(f"router linear T={T} H={H} E={E}", flush=True)
    g = torch.Generator().manual_seed(T + E + H)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    ref = x.float() @ wr.float().t()
    out32 = ops.router_linear(x, wr, torch.float32)
    out16 = ops.router_linear(x, wr, torch.bfloat16)
    torch.cuda.synchronize()
    assert out32.dtype == torch.float32 and out16.dtype == torch.bfloat16
    assert _rel(out32, ref) < 1e-5
    # bf16: |out16 - ref| <= half an ulp of bf16 at the value plus the fp32 noise
    err = (out16.double() - ref.double()).abs()
    bound = ref.double().abs() * 2.0 ** -8 + 1e-5 * ref.abs().max().item()
    assert bool((err <= bound).all())


def test_router_linear_rejects():
    x = torch.zeros(64, 96, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        ops.router_linear(x, torch.zeros(8, 96, dtype=torch.bfloat16, device=DEV))
    x = torch.zeros(64, 128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="of 8"):
        ops.router_linear(x, torch.zeros(12, 128, dtype=torch.bfloat16, device=DEV))
    with pytest.raises(TypeError):
        ops.router_linear(x.float(), torch.zeros(8, 128, device=DEV))


def test_router_linear_zero_tokens():
    """No tokens: empty logits and an empty dX, no error."""
    x = torch.empty(0, 256, dtype=torch.bfloat16, device=DEV)
    wr = torch.randn(16, 256, device=DEV).to(torch.bfloat16)
    assert ops.router_linear(x, wr, torch.float32).shape == (0, 16)
    assert ops.router_linear(x, wr, torch.bfloat16).shape == (0, 16)
    dl = torch.empty(0, 16, dtype=torch.bfloat16, device=DEV)
    assert ops.router_linear_backward_dx(dl, wr).shape == (0, 256)
    dw = ops.router_linear_backward_dw(dl, x)
    torch.cuda.synchronize()
    assert dw.shape == (16, 256) and not dw.any()


@pytest.mark.parametrize("router", ["softmax", "sigmoid"])
@pytest.mark.parametrize("E,K,dtype", [(128, 8, torch.bfloat16), (1792, 8, torch.float32),
                                       (600, 6, torch.bfloat16)])
def test_router_nan_rows(router, E, K, dtype):
    """Rows holding NaN logits (of either sign) route exactly as the oracle:
    valid expert ids always (never a placeholder), NaN ranked above every
    number; for the softmax router a NaN makes the whole prob row NaN, so
    the K lowest ids are chosen; on the E > 256 wave-per-token kernels as on
    the group kernels."""
    print(f"NaN rows {router} E={E} K={K} {dtype}", flush=True)
    g = torch.Generator().manual_seed(E + K)
    T = 64
    logits = torch.randn(T, E, generator=g)
    logits[3, 7] = float("nan")
    logits[5, E - 1] = -float("nan")
    logits[9, :] = float("nan")
    logits[11, ::2] = float("nan")
    if router == "softmax":
        lg = logits.to(dtype).to(DEV)
        probs, w, idx = ops.router_softmax_topk(lg, K, True)
        p_ref, w_ref, i_ref = O.softmax_router(lg.cpu(), K)
    else:
        lg = logits.to(DEV)
        bias = ((torch.rand(E, generator=g) * 2 - 1) * 0.5).to(DEV)
        probs, w, idx = ops.router_sigmoid_topk(lg, bias, K, True, None, None, None,
                                                torch.float32)
        p_ref, w_ref, i_ref = O.sigmoid_router(lg.cpu(), bias.cpu(), K)
    torch.cuda.synchronize()
    ic = idx.cpu()
    assert bool(((ic >= 0) & (ic < E)).all()), "invalid expert id"
    assert torch.equal(ic, i_ref)
    nan_rows = torch.isnan(logits).any(-1)
    assert torch.equal(torch.isnan(w.cpu()).any(-1), nan_rows)
    ok = ~nan_rows
    assert torch.allclose(w.cpu()[ok], w_ref[ok], rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("T,H,E,K,with_off", [
    (65536, 2048, 128, 8, False),   # L / M shape, full token count
    (16384, 1024, 128, 4, True),    # XS global bank with the logit offset
    (1000, 256, 256, 12, True),     # 16 lanes per token, K > 8
    (777, 128, 200, 8, False),      # 16 lanes per token, partly empty lanes, ragged T
    (333, 192, 72, 6, True),        # 8 lanes per token, mostly empty lanes, ragged T
    (5, 64, 136, 16, False),        # fewer tokens than one tile, K = 16
])
def test_router_fused_softmax_topk(T, H, E, K, with_off):
    """The gating linear with the softmax router in its epilogue equals the
    two-kernel form (router_linear bf16 -> router_softmax_topk) bit for bit --
    probabilities, weights, ids and the logits it writes -- and the oracle's
    routing on those logits exactly."""
    print(f"fused router T={T} H={H} E={E} K={K} offset={with_off}", flush=True)
    g = torch.Generator().manual_seed(T + E + K)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV)
    wr = (torch.randn(E, H, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    off = ((torch.rand(E, generator=g) * 2 - 1) * 0.5).to(DEV) if with_off else None
    for renorm in (True, False):
        probs, w, idx, lg = ops.router_linear_softmax_topk(x, wr, K, renorm, off,
                                                          return_logits=True)
        logits = ops.router_linear(x, wr, torch.bfloat16)
        p2, w2, i2 = ops.router_softmax_topk(logits, K, renorm, off)
        p3, w3, i3 = ops.router_linear_softmax_topk(x, wr, K, renorm, off)
        torch.cuda.synchronize()
        assert torch.equal(lg, logits), "fused logits differ from router_linear's"
        assert torch.equal(idx, i2) and torch.equal(i3, i2), "fused routing ids differ"
        for a, b in ((probs, p2), (w, w2), (p3, p2), (w3, w2)):
            assert torch.equal(a.view(torch.int32), b.view(torch.int32)), "fused values differ"
        if T <= 20000:
            p_ref, w_ref, i_ref = O.softmax_router(logits.cpu(), K, renorm,
                                                   None if off is None else off.cpu())
            assert torch.equal(idx.cpu(), i_ref)
            assert torch.allclose(probs.cpu(), p_ref, rtol=1e-5, atol=1e-7)
            assert torch.allclose(w.cpu(), w_ref, rtol=1e-5, atol=1e-7)


def test_router_fused_nan_rows_and_rejects():
    """A NaN hidden state makes its token's logits NaN: the fused router
    routes it as the two-kernel form does (the K lowest ids); shapes outside
    the fused kernel's are refused with the two-kernel form named."""
    g = torch.Generator().manual_seed(5)
    T, H, E, K = 300, 128, 128, 8
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    x[7, 3] = float("nan")
    x, wr = x.to(DEV), (torch.randn(E, H, generator=g) * 0.05).to(torch.bfloat16).to(DEV)
    probs, w, idx = ops.router_linear_softmax_topk(x, wr, K)
    p2, w2, i2 = ops.router_softmax_topk(ops.router_linear(x, wr, torch.bfloat16), K)
    torch.cuda.synchronize()
    assert torch.equal(idx, i2) and idx[7].tolist() == list(range(K))
    assert torch.equal(probs.view(torch.int32), p2.view(torch.int32))
    assert torch.equal(w.view(torch.int32), w2.view(torch.int32))
    for e, k in ((64, 4), (1792, 8), (128, 9)):
        wbad = torch.zeros(e, H, dtype=torch.bfloat16, device=DEV)
        with pytest.raises(RuntimeError, match="router_softmax_topk"):
            ops.router_linear_softmax_topk(x, wbad, k)
    assert ops.router_linear_softmax_topk(x[:0], wr, K)[2].shape == (0, K)


@pytest.mark.parametrize("T,H,E,fp32", [(512, 2048, 1792, True), (1000, 256, 128, False),
                                        (300, 192, 72, True)])
def test_torch_gating_linear_op(T, H, E, fp32):
    """The torch-forward gating op: logits bit-identical to torch's own
    F.linear (the reference's routing input), gradients from the MFMA
    backward within one bf16 rounding of the fp64 chain rule (torch's own
    fp32 fallback where the MFMA shapes do not apply)."""
    from moe_amd.router import gating_linear
    print(f"torch gating op T={T} H={H} E={E} fp32={fp32}", flush=True)
    g = torch.Generator().manual_seed(T + E)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(DEV).requires_grad_(True)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16).to(DEV).requires_grad_(True)
    lg = gating_linear(x, wr, fp32, hip=False)
    ref = F.linear(x.detach().float(), wr.detach().float()) if fp32 else F.linear(x.detach(),
                                                                                  wr.detach())
    assert lg.dtype == ref.dtype and torch.equal(lg, ref), "logits differ from torch's F.linear"
    dl = torch.randn(T, E, generator=g).to(lg.dtype).to(DEV)
    lg.backward(dl)
    dx_ref = dl.double() @ wr.detach().double()
    dw_ref = dl.double().t() @ x.detach().double()
    assert _rel(x.grad, dx_ref) < 1e-2 and _rel(wr.grad, dw_ref) < 1e-2
