"""torch.library registrations of the HIP expert layer and routers.

The reference's experts backend registers its grouped GEMM as a custom op
with a fake (shape) implementation and an autograd formula
(transformers/integrations/moe.py:245-257), so that torch.compile traces the
layer without a graph break.  The same contract holds here for every
differentiable piece of the MI355X path, each a functional op in namespace
``moe_amd``:

  experts_fwd / experts_bwd      the expert layer (permute, GEMM-1 + SwiGLU,
                                 GEMM-2, combine; fused backward)
  moe_layer_fwd / moe_layer_bwd  gating linear + softmax router + experts as
                                 one node (the two hidden-state gradients meet
                                 inside the gather backward)
  router_linear / _backward      the gating linear on the MFMA kernel
  softmax_topk / _backward       Qwen3MoeTopKRouter's softmax + top-k
  sigmoid_topk / _backward       DeepSeekRouter's sigmoid + biased top-k
  linear_sigmoid_topk            its fp32 gating linear and the router in one
                                 kernel (backward: sigmoid_topk_backward, then
                                 router_linear_backward)

A forward op returns, besides its results, the tensors its backward needs
(the routing plan, gate_up), so that setup_context saves only op outputs; the
public functions in experts.py, router.py and layer.py return the results.
Ops run their HIP entry points on torch's current stream; the fake
implementations only compute output shapes (the tile plan's byte size is a
host function of S and E, or an unbacked size under symbolic shapes).
Gradients that a caller does not need come back as empty tensors from the
backward ops and as None from autograd.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _lib, ops

_LIB = "moe_amd"


def _plan_bytes(S, E) -> int:
    if isinstance(S, int) and isinstance(E, int):
        return int(_lib.load().moe_amd_tile_plan_size(S, E))
    return torch.library.get_ctx().new_dynamic_size()


def _plan_fake(S, E, dev):
    i32 = dict(device=dev, dtype=torch.int32)
    return (torch.empty(E, **i32), torch.empty(E + 1, **i32), torch.empty(S, **i32),
            torch.empty(S, **i32), torch.empty(_plan_bytes(S, E), device=dev, dtype=torch.uint8))


def _plan(counts, offsets, row_src, slot, tile_plan, E, K, T) -> ops.RoutingPlan:
    return ops.RoutingPlan(counts, offsets, row_src, slot, tile_plan, E, K, T)


def _empty_like_none(t: Tensor) -> Tensor:
    return t.new_empty(0)


def _main_grad(weight: Tensor) -> Optional[Tensor]:
    """The fused gradient-accumulation buffer of an expert weight: its
    ``main_grad`` attribute (Megatron-LM's name for it), or None.  When set,
    the layer's backward adds the weight's gradient into it in place (with
    the bits autograd's accumulation would give) and hands autograd None for
    the weight; experts without routed rows are not touched, so an expert
    bank shared by several layers is never written whole.  bf16 weights and
    a bf16, contiguous main_grad of the weight's shape on its device only."""
    g = getattr(weight, "main_grad", None)
    if g is None:
        return None
    if (not isinstance(g, Tensor) or weight.dtype != torch.bfloat16 or g.dtype != torch.bfloat16
            or g.shape != weight.shape or g.device != weight.device or not g.is_contiguous()):
        raise ValueError("main_grad: fused gradient accumulation takes a bf16 expert weight and "
                         "a contiguous bf16 main_grad of its shape on its device")
    return g


# ------------------------------------------------------------------ experts

def _saves_act_y(dtype: torch.dtype, save_for_backward: bool) -> bool:
    # The fp32 layer's backward is the unfused one (combine backward, then
    # GEMM-2's dX / dW from d_y): it needs act and y; bf16 recomputes act
    # from gate_up inside its fused backward and needs neither.
    return save_for_backward and dtype == torch.float32


@torch.library.custom_op(f"{_LIB}::experts_fwd", mutates_args=())
def experts_fwd(hidden_states: Tensor, top_k_index: Tensor, top_k_weights: Tensor,
                gate_up_proj: Tensor, down_proj: Tensor, save_for_backward: bool
                ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                           Tensor]:
    """(out [T,H], gate_up [S,2I] or [0,2I], act [S,I] and y [S,H] (fp32
    with save_for_backward; else [0,I], [0,H]), counts, offsets, row_src,
    slot, tile_plan).  transformers/integrations/moe.py:377-478."""
    plan = ops.permute(top_k_index, gate_up_proj.shape[0])
    gu, act = ops.gemm_gate_up_swiglu(hidden_states, plan, gate_up_proj,
                                      save_gate_up=save_for_backward)
    y = ops.gemm_down(act, plan, down_proj)
    out = ops.combine(y, plan, top_k_weights)
    if not _saves_act_y(hidden_states.dtype, save_for_backward):
        act, y = act.new_empty(0, act.shape[1]), y.new_empty(0, y.shape[1])
    if gu is None:
        gu = hidden_states.new_empty(0, gate_up_proj.shape[1])
    return out, gu, act, y, plan.counts, plan.offsets, plan.row_src, plan.slot, plan.tile_plan


@experts_fwd.register_fake
def _(hidden_states, top_k_index, top_k_weights, gate_up_proj, down_proj, save_for_backward):
    T, H = hidden_states.shape
    S = T * top_k_index.shape[1]
    E, I2 = gate_up_proj.shape[0], gate_up_proj.shape[1]
    out = hidden_states.new_empty(T, H)
    gu = hidden_states.new_empty(S if save_for_backward else 0, I2)
    sa = S if _saves_act_y(hidden_states.dtype, save_for_backward) else 0
    act, y = hidden_states.new_empty(sa, I2 // 2), hidden_states.new_empty(sa, H)
    return (out, gu, act, y) + _plan_fake(S, E, hidden_states.device)


_SIDE_STREAMS: dict = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """A second stream per device (default priority), created once."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    s = _SIDE_STREAMS.get(idx)
    if s is None:
        s = _SIDE_STREAMS[idx] = torch.cuda.Stream(device=idx)
    return s


def _gather_backward_beside(d_xs: Tensor, plan, addend: Optional[Tensor]):
    """d_x = gather_backward(d_xs, plan, addend) launched on a second stream,
    after the current stream's work so far, so that it (HBM-bound, no LDS)
    runs beside the weight-gradient GEMMs the caller launches next (MFMA-
    bound, one workgroup per CU holding all of its LDS and 376-380 of each
    SIMD's 512 VGPRs per lane; the gather needs no LDS and at most 62 VGPRs, so
    its waves share those CUs).  Returns (d_x, join): join() makes the current
    stream wait for it.  With per-launch timing on, it runs in order instead."""
    if ops.kernel_timing_active():
        return ops.gather_backward(d_xs, plan, addend=addend), lambda: None
    main = torch.cuda.current_stream(d_xs.device)
    side = _side_stream(d_xs.device)
    side.wait_stream(main)
    with torch.cuda.stream(side):
        d_x = ops.gather_backward(d_xs, plan, addend=addend)
    for t in (d_xs, addend, plan.counts, plan.offsets, plan.row_src, plan.slot, plan.tile_plan):
        if t is not None:
            t.record_stream(side)
    d_x.record_stream(main)
    return d_x, lambda: main.wait_stream(side)


def _experts_bwd_f32(d_out, x, w, w1, w2, gu, act, y, plan, need_x, need_w1, need_w2):
    """fp32: the reference's autograd chain kernel by kernel (combine
    backward -> GEMM-2 dX + dSwiGLU, GEMM-2 dW -> GEMM-1 dW, dX -> gather
    backward), every product and sum in fp32."""
    dy, dw = ops.combine_backward(d_out, y, plan, w)
    d_gu = ops.gemm_down_backward_dx_dswiglu(dy, plan, w2, gu)
    d_w2 = ops.gemm_down_backward_dw(dy, act, plan, w2.shape) if need_w2 else w2.new_empty(0)
    del dy
    d_w1 = (ops.gemm_gate_up_backward_dw(d_gu, x, plan, w1.shape) if need_w1
            else w1.new_empty(0))
    d_x = (ops.gather_backward(ops.gemm_gate_up_backward_dx(d_gu, plan, w1), plan) if need_x
           else x.new_empty(0))
    return d_x, dw, d_w1, d_w2


def _dw_down(d_out, act_w, plan, down_proj, need, acc):
    if not need:
        return _empty_like_none(down_proj)
    if acc is not None:
        ops.gemm_down_backward_dw_gathered_accumulate(d_out, act_w, plan, acc)
        return _empty_like_none(down_proj)
    return ops.gemm_down_backward_dw_gathered(d_out, act_w, plan, down_proj.shape)


def _dw_gate_up(d_gu, x, plan, gate_up_proj, need, acc):
    if not need:
        return _empty_like_none(gate_up_proj)
    if acc is not None:
        ops.gemm_gate_up_backward_dw_accumulate(d_gu, x, plan, acc)
        return _empty_like_none(gate_up_proj)
    return ops.gemm_gate_up_backward_dw(d_gu, x, plan, gate_up_proj.shape)


@torch.library.custom_op(f"{_LIB}::experts_bwd", mutates_args=("acc_w1", "acc_w2"))
def experts_bwd(d_out: Tensor, hidden_states: Tensor, top_k_weights: Tensor, gate_up_proj: Tensor,
                down_proj: Tensor, gate_up: Tensor, act: Tensor, y: Tensor, counts: Tensor,
                offsets: Tensor, row_src: Tensor, slot: Tensor, tile_plan: Tensor, need_x: bool,
                need_w1: bool, need_w2: bool, acc_w1: Optional[Tensor],
                acc_w2: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(d_x, d_topk_weights, d_gate_up_proj, d_down_proj) (formulas
    integrations/moe.py:226-242).  bf16: the combine's backward runs fused
    into GEMM-2's; fp32: the unfused chain on the saved act and y.  With
    acc_w1 / acc_w2 (bf16 only) the weight gradients are added into them in
    place and returned empty."""
    T, K = top_k_weights.shape
    plan = _plan(counts, offsets, row_src, slot, tile_plan, gate_up_proj.shape[0], K, T)
    d_out = d_out.to(hidden_states.dtype).contiguous()
    if hidden_states.dtype == torch.float32:
        if acc_w1 is not None or acc_w2 is not None:
            raise ValueError("experts_bwd: fused gradient accumulation takes bf16 layers only")
        return _experts_bwd_f32(d_out, hidden_states, top_k_weights.contiguous(), gate_up_proj,
                                down_proj, gate_up, act, y, plan, need_x, need_w1, need_w2)
    d_gu, act_w, dw = ops.gemm_down_backward_fused(d_out, plan, down_proj, gate_up, top_k_weights)
    join = None
    if need_x:
        d_x, join = _gather_backward_beside(
            ops.gemm_gate_up_backward_dx(d_gu, plan, gate_up_proj), plan, None)
    else:
        d_x = _empty_like_none(hidden_states)
    d_w2 = _dw_down(d_out, act_w, plan, down_proj, need_w2, acc_w2)
    del act_w
    d_w1 = _dw_gate_up(d_gu, hidden_states, plan, gate_up_proj, need_w1, acc_w1)
    if join is not None:
        join()
    return d_x, dw, d_w1, d_w2


@experts_bwd.register_fake
def _(d_out, hidden_states, top_k_weights, gate_up_proj, down_proj, gate_up, act, y, counts,
      offsets, row_src, slot, tile_plan, need_x, need_w1, need_w2, acc_w1, acc_w2):
    return (torch.empty_like(hidden_states) if need_x else hidden_states.new_empty(0),
            torch.empty_like(top_k_weights),
            torch.empty_like(gate_up_proj) if need_w1 and acc_w1 is None
            else gate_up_proj.new_empty(0),
            torch.empty_like(down_proj) if need_w2 and acc_w2 is None
            else down_proj.new_empty(0))


def _experts_setup(ctx, inputs, output):
    x, _, w, w1, w2, _ = inputs
    _, gu, act, y, counts, offsets, row_src, slot, tile_plan = output
    # The saved activations are outputs only for saving: no zero [S, 2I]
    # gradient is materialised for them.
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(x, w, w1, w2, gu, act, y, counts, offsets, row_src, slot, tile_plan)
    ctx.main_grads = (_main_grad(w1), _main_grad(w2))


def _experts_backward(ctx, d_out, *unused):
    need_x, _, need_w, need_w1, need_w2 = ctx.needs_input_grad[:5]
    if d_out is None:
        return (None,) * 6
    acc1, acc2 = ctx.main_grads
    d_x, d_w, d_w1, d_w2 = torch.ops.moe_amd.experts_bwd(
        d_out, *ctx.saved_tensors, bool(need_x), bool(need_w1), bool(need_w2),
        acc1 if need_w1 else None, acc2 if need_w2 else None)
    return (d_x if need_x else None, None, d_w if need_w else None,
            d_w1 if need_w1 and acc1 is None else None,
            d_w2 if need_w2 and acc2 is None else None, None)


torch.library.register_autograd(f"{_LIB}::experts_fwd", _experts_backward,
                                setup_context=_experts_setup)


# ----------------------------------------------------------- gating linear

@torch.library.custom_op(f"{_LIB}::router_linear", mutates_args=())
def router_linear(x: Tensor, weight: Tensor, out_dtype: torch.dtype) -> Tensor:
    """logits = x . W^T, fp32 accumulation, logits in out_dtype (bf16:
    src/models/modeling_qwen3_moe.py:268-270; fp32: src/models/router.py:107-109)."""
    return ops.router_linear(x, weight, out_dtype)


@router_linear.register_fake
def _(x, weight, out_dtype):
    return x.new_empty(x.shape[0], weight.shape[0], dtype=out_dtype)


@torch.library.custom_op(f"{_LIB}::router_linear_backward", mutates_args=())
def router_linear_backward(d_logits: Tensor, x: Tensor, weight: Tensor, out_dtype: torch.dtype,
                           need_x: bool, need_w: bool) -> tuple[Tensor, Tensor]:
    """(d_x, d_W).  bf16 logits: the MFMA dX and split-K dW kernels (fp32
    accumulation, one bf16 rounding, as F.linear's bf16 backward); fp32
    logits (the DeepSeek router's fp32 linear): the same kernels on a
    two-term bf16 split of d_logits, fp32-accurate, each gradient rounded
    once to the inputs' bf16.  H a multiple of 256 (and E of 32 for fp32
    logits), else torch on the same device in the logits' precision."""
    E, H = weight.shape
    dx = x.new_empty(0)
    dw = weight.new_empty(0)
    bf = x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
    if out_dtype == torch.float32:
        g = d_logits.float()
        if bf and H % 256 == 0 and E % 32 == 0:
            return ops.router_linear_backward_f32(g, x, weight, need_x, need_w)
        if need_x:
            dx = (g @ weight.float()).to(x.dtype)
        if need_w:
            dw = (g.t().contiguous() @ x.float()).to(weight.dtype)
    else:
        g = d_logits.to(x.dtype)
        if need_x:
            dx = ops.router_linear_backward_dx(g, weight) if H % 256 == 0 else g @ weight
        if need_w:
            dw = (ops.router_linear_backward_dw(g, x) if H % 256 == 0
                  else g.t().contiguous() @ x)
    return dx, dw


@router_linear_backward.register_fake
def _(d_logits, x, weight, out_dtype, need_x, need_w):
    return (torch.empty_like(x) if need_x else x.new_empty(0),
            torch.empty_like(weight) if need_w else weight.new_empty(0))


def _linear_setup(ctx, inputs, output):
    x, weight, out_dtype = inputs
    ctx.save_for_backward(x, weight)
    ctx.out_dtype = out_dtype


def _linear_backward(ctx, d_logits):
    x, weight = ctx.saved_tensors
    need_x, need_w = ctx.needs_input_grad[:2]
    dx, dw = torch.ops.moe_amd.router_linear_backward(d_logits, x, weight, ctx.out_dtype,
                                                      bool(need_x), bool(need_w))
    return (dx if need_x else None, dw if need_w else None, None)


torch.library.register_autograd(f"{_LIB}::router_linear", _linear_backward,
                                setup_context=_linear_setup)


@torch.library.custom_op(f"{_LIB}::torch_gating_linear", mutates_args=())
def torch_gating_linear(x: Tensor, weight: Tensor, fp32: bool) -> Tensor:
    """The reference's gating linear computed by torch itself (F.linear(x, W),
    or F.linear(x.float(), W.float()) for the DeepSeek router), so the logits
    and the routing are the reference's bit for bit; its backward is the MFMA
    kernels' (router_linear_backward: fp32 accumulation, one rounding per
    gradient)."""
    return ops.torch_gating_linear(x, weight, fp32)


@torch_gating_linear.register_fake
def _(x, weight, fp32):
    return x.new_empty(x.shape[0], weight.shape[0],
                       dtype=torch.float32 if fp32 else x.dtype)


def _torch_gating_setup(ctx, inputs, output):
    x, weight, fp32 = inputs
    ctx.save_for_backward(x, weight)
    ctx.out_dtype = torch.float32 if fp32 else x.dtype


torch.library.register_autograd(f"{_LIB}::torch_gating_linear", _linear_backward,
                                setup_context=_torch_gating_setup)


# ---------------------------------------------------------- softmax router

@torch.library.custom_op(f"{_LIB}::softmax_topk", mutates_args=())
def softmax_topk(logits: Tensor, top_k: int, renormalize: bool,
                 logit_offset: Optional[Tensor]) -> tuple[Tensor, Tensor, Tensor]:
    """(probs fp32 [T,E], weights fp32 [T,K], index int64 [T,K]);
    src/models/modeling_qwen3_moe.py:266-275."""
    return ops.router_softmax_topk(logits, top_k, renormalize, logit_offset)


@softmax_topk.register_fake
def _(logits, top_k, renormalize, logit_offset):
    T, E = logits.shape
    f32 = dict(device=logits.device, dtype=torch.float32)
    return (torch.empty(T, E, **f32), torch.empty(T, top_k, **f32),
            torch.empty(T, top_k, device=logits.device, dtype=torch.int64))


@torch.library.custom_op(f"{_LIB}::softmax_topk_backward", mutates_args=())
def softmax_topk_backward(probs: Tensor, topk_index: Tensor, d_weights: Optional[Tensor],
                          d_probs: Optional[Tensor], renormalize: bool,
                          logits_dtype: torch.dtype) -> Tensor:
    """d_logits [T,E] in the logits' dtype (autograd of :266-275)."""
    if d_weights is None:
        d_weights = torch.zeros(topk_index.shape, device=probs.device, dtype=torch.float32)
    return ops.router_softmax_topk_backward(probs, topk_index, d_weights, d_probs, renormalize,
                                            logits_dtype)


@softmax_topk_backward.register_fake
def _(probs, topk_index, d_weights, d_probs, renormalize, logits_dtype):
    return torch.empty_like(probs, dtype=logits_dtype)


def _softmax_setup(ctx, inputs, output):
    logits, _, renormalize, _ = inputs
    probs, _, idx = output
    ctx.set_materialize_grads(False)
    ctx.mark_non_differentiable(idx)
    ctx.save_for_backward(probs, idx)
    ctx.renormalize = renormalize
    ctx.logits_dtype = logits.dtype


def _softmax_backward(ctx, d_probs, d_w, d_idx):
    probs, idx = ctx.saved_tensors
    if d_probs is None and d_w is None:
        return None, None, None, None
    d_logits = torch.ops.moe_amd.softmax_topk_backward(probs, idx, d_w, d_probs, ctx.renormalize,
                                                       ctx.logits_dtype)
    return d_logits, None, None, None


torch.library.register_autograd(f"{_LIB}::softmax_topk", _softmax_backward,
                                setup_context=_softmax_setup)


# --------------------------------------------------------- DeepSeek router

@torch.library.custom_op(f"{_LIB}::sigmoid_topk", mutates_args=())
def sigmoid_topk(logits: Tensor, expert_bias: Optional[Tensor], top_k: int, renormalize: bool,
                 scaling_factor: float, num_groups: int, group_topk: int,
                 weights_dtype: torch.dtype, count: bool
                 ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(scores fp32 [T,E], weights [T,K] in weights_dtype, index int64 [T,K],
    selection counts fp32 [E] (zeros unless count)); src/models/router.py:
    103-155.  scaling_factor 0 = none; num_groups/group_topk 0 = flat top-k.
    The counts come back as an output (the op is functional); the router adds
    them to its local_tokens_per_expert buffer."""
    counts = torch.zeros(logits.shape[1], device=logits.device, dtype=torch.float32)
    if logits.dtype == torch.float32:
        scores, w, idx = ops.router_sigmoid_topk(
            logits, expert_bias, top_k, renormalize, scaling_factor or None,
            num_groups or None, group_topk or None, weights_dtype, counts if count else None)
    else:
        # bf16 logits: the reference under bf16 autocast, whose fp32 gating
        # linear still yields bf16 logits; its torch.sigmoid then gives bf16
        # scores (router.py:112), computed here by the same torch call.
        scores = torch.sigmoid(logits)
        w, idx = ops.router_sigmoid_topk_scores(
            scores, expert_bias, top_k, renormalize, scaling_factor or None,
            num_groups or None, group_topk or None, weights_dtype, counts if count else None)
    return scores, w, idx, counts


@sigmoid_topk.register_fake
def _(logits, expert_bias, top_k, renormalize, scaling_factor, num_groups, group_topk,
      weights_dtype, count):
    T, E = logits.shape
    dev = logits.device
    return (torch.empty(T, E, device=dev, dtype=logits.dtype),
            torch.empty(T, top_k, device=dev, dtype=weights_dtype),
            torch.empty(T, top_k, device=dev, dtype=torch.int64),
            torch.empty(E, device=dev, dtype=torch.float32))


@torch.library.custom_op(f"{_LIB}::sigmoid_topk_backward", mutates_args=())
def sigmoid_topk_backward(scores: Tensor, topk_index: Tensor, d_weights: Tensor,
                          d_scores: Optional[Tensor], renormalize: bool,
                          scaling_factor: float) -> Tensor:
    """d_logits [T,E] in the scores' dtype (autograd of router.py:112-140)."""
    return ops.router_sigmoid_topk_backward(scores, topk_index, d_weights, d_scores, renormalize,
                                            scaling_factor or None).to(scores.dtype)


@sigmoid_topk_backward.register_fake
def _(scores, topk_index, d_weights, d_scores, renormalize, scaling_factor):
    return torch.empty_like(scores)


def _sigmoid_setup(ctx, inputs, output):
    _, _, _, renormalize, scaling_factor, _, _, weights_dtype, _ = inputs
    scores, _, idx, counts = output
    ctx.set_materialize_grads(False)
    ctx.mark_non_differentiable(idx, counts)
    ctx.save_for_backward(scores, idx)
    ctx.renormalize = renormalize
    ctx.scaling_factor = scaling_factor
    ctx.w_dtype = weights_dtype


def _sigmoid_backward(ctx, d_scores, d_w, d_idx, d_counts):
    scores, idx = ctx.saved_tensors
    none = (None,) * 8
    if d_scores is None and d_w is None:
        return (None,) + none
    if d_w is None:
        d_w = torch.zeros(idx.shape, device=idx.device, dtype=ctx.w_dtype)
    d_logits = torch.ops.moe_amd.sigmoid_topk_backward(scores, idx, d_w.to(ctx.w_dtype), d_scores,
                                                       ctx.renormalize, ctx.scaling_factor)
    return (d_logits,) + none


torch.library.register_autograd(f"{_LIB}::sigmoid_topk", _sigmoid_backward,
                                setup_context=_sigmoid_setup)


@torch.library.custom_op(f"{_LIB}::linear_sigmoid_topk", mutates_args=())
def linear_sigmoid_topk(x: Tensor, w_router: Tensor, expert_bias: Optional[Tensor], top_k: int,
                        renormalize: bool, scaling_factor: float, num_groups: int,
                        group_topk: int, weights_dtype: torch.dtype, count: bool
                        ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The DeepSeek router with its fp32 gating linear in one kernel: (scores
    fp32 [T,E], weights [T,K], index [T,K], selection counts fp32 [E] (zeros
    unless count)); the same bits as router_linear(fp32) + sigmoid_topk
    (src/models/router.py:103-152)."""
    counts = torch.zeros(w_router.shape[0], device=x.device, dtype=torch.float32)
    scores, w, idx = ops.router_linear_sigmoid_topk(
        x, w_router, expert_bias, top_k, renormalize, scaling_factor or None,
        num_groups or None, group_topk or None, weights_dtype, counts if count else None)
    return scores, w, idx, counts


@linear_sigmoid_topk.register_fake
def _(x, w_router, expert_bias, top_k, renormalize, scaling_factor, num_groups, group_topk,
      weights_dtype, count):
    T, E = x.shape[0], w_router.shape[0]
    dev = x.device
    return (torch.empty(T, E, device=dev, dtype=torch.float32),
            torch.empty(T, top_k, device=dev, dtype=weights_dtype),
            torch.empty(T, top_k, device=dev, dtype=torch.int64),
            torch.empty(E, device=dev, dtype=torch.float32))


def _linear_sigmoid_setup(ctx, inputs, output):
    x, w_router, _, _, renormalize, scaling_factor, _, _, weights_dtype, _ = inputs
    scores, _, idx, counts = output
    ctx.set_materialize_grads(False)
    ctx.mark_non_differentiable(idx, counts)
    ctx.save_for_backward(x, w_router, scores, idx)
    ctx.renormalize = renormalize
    ctx.scaling_factor = scaling_factor
    ctx.w_dtype = weights_dtype


def _linear_sigmoid_backward(ctx, d_scores, d_w, d_idx, d_counts):
    """The router's backward (sigmoid_topk_backward: gather, renormalisation,
    scaling, sigmoid) into the fp32 gating linear's two gradients."""
    x, w_router, scores, idx = ctx.saved_tensors
    need_x, need_wr = (bool(n) for n in ctx.needs_input_grad[:2])
    none = (None,) * 8
    if (d_scores is None and d_w is None) or not (need_x or need_wr):
        return (None, None) + none
    if d_w is None:
        d_w = torch.zeros(idx.shape, device=idx.device, dtype=ctx.w_dtype)
    d_logits = torch.ops.moe_amd.sigmoid_topk_backward(scores, idx, d_w.to(ctx.w_dtype), d_scores,
                                                       ctx.renormalize, ctx.scaling_factor)
    dx, dw = torch.ops.moe_amd.router_linear_backward(d_logits, x, w_router, torch.float32,
                                                      need_x, need_wr)
    return (dx if need_x else None, dw if need_wr else None) + none


torch.library.register_autograd(f"{_LIB}::linear_sigmoid_topk", _linear_sigmoid_backward,
                                setup_context=_linear_sigmoid_setup)


# ------------------------------------------------ softmax layer, one node

GATINGS = ("torch", "hip", "hip_fused")


def gating_logits(x: Tensor, w_router: Tensor, gating: str, fp32: bool) -> Tensor:
    """Router logits from the gating source ``gating``: "torch" = the
    reference's F.linear on this device (bit-identical logits, hence the
    reference's routing), "hip" = the MFMA gating-linear kernel (same exact
    products, its own fp32 summation order); "hip_fused" computes the same
    logits as "hip" (the softmax router then runs in the kernel's
    epilogue)."""
    if gating == "torch":
        return ops.torch_gating_linear(x, w_router, fp32)
    if gating in ("hip", "hip_fused"):
        return ops.router_linear(x, w_router, torch.float32 if fp32 else torch.bfloat16)
    raise ValueError(f"unknown gating {gating!r} (expected one of {GATINGS})")


@torch.library.custom_op(f"{_LIB}::moe_layer_fwd", mutates_args=())
def moe_layer_fwd(x: Tensor, w_router: Tensor, gate_up_proj: Tensor, down_proj: Tensor,
                  top_k: int, renormalize: bool, logit_offset: Optional[Tensor],
                  save_for_backward: bool, gating: str
                  ) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                             Tensor, Tensor]:
    """(out, probs fp32, weights fp32, index, gate_up, counts, offsets, row_src,
    slot, tile_plan): bf16 gating linear (source ``gating``), softmax router,
    experts (Qwen3MoeSparseMoeBlock.forward, src/models/modeling_qwen3_moe.py:
    284-289).  The backward runs the gating linear's gradients on the MFMA
    kernels whichever source computed the logits."""
    if gating == "hip_fused" and ops.router_fused_supported(w_router.shape[0], top_k):
        # gating linear + softmax router in one kernel (same bits as "hip")
        probs, w, idx = ops.router_linear_softmax_topk(x, w_router, top_k, renormalize,
                                                       logit_offset)
    else:
        logits = gating_logits(x, w_router, gating, fp32=False)
        probs, w, idx = ops.router_softmax_topk(logits, top_k, renormalize, logit_offset)
        del logits
    plan = ops.permute(idx, gate_up_proj.shape[0])
    gu, act = ops.gemm_gate_up_swiglu(x, plan, gate_up_proj, save_gate_up=save_for_backward)
    y = ops.gemm_down(act, plan, down_proj)
    del act
    out = ops.combine(y, plan, w)
    if gu is None:
        gu = x.new_empty(0, gate_up_proj.shape[1])
    return (out, probs, w, idx, gu, plan.counts, plan.offsets, plan.row_src, plan.slot,
            plan.tile_plan)


@moe_layer_fwd.register_fake
def _(x, w_router, gate_up_proj, down_proj, top_k, renormalize, logit_offset, save_for_backward,
      gating):
    T, H = x.shape
    E, I2 = gate_up_proj.shape[0], gate_up_proj.shape[1]
    S = T * top_k
    dev = x.device
    f32 = dict(device=dev, dtype=torch.float32)
    return (x.new_empty(T, H), torch.empty(T, E, **f32), torch.empty(T, top_k, **f32),
            torch.empty(T, top_k, device=dev, dtype=torch.int64),
            x.new_empty(S if save_for_backward else 0, I2)) + _plan_fake(S, E, dev)


@torch.library.custom_op(f"{_LIB}::moe_layer_bwd", mutates_args=("acc_w1", "acc_w2"))
def moe_layer_bwd(d_out: Optional[Tensor], d_probs: Optional[Tensor], d_w: Optional[Tensor],
                  x: Tensor, w_router: Tensor, gate_up_proj: Tensor, down_proj: Tensor,
                  gate_up: Tensor, probs: Tensor, w: Tensor, idx: Tensor, counts: Tensor,
                  offsets: Tensor, row_src: Tensor, slot: Tensor, tile_plan: Tensor,
                  renormalize: bool, need_x: bool, need_wr: bool, need_w1: bool, need_w2: bool,
                  acc_w1: Optional[Tensor], acc_w2: Optional[Tensor]
                  ) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(d_x, d_w_router, d_gate_up_proj, d_down_proj).  The combine backward
    runs fused into GEMM-2's; the gating linear's dX is added inside the
    gather backward.  acc_w1 / acc_w2: as for experts_bwd."""
    T, K = idx.shape
    plan = _plan(counts, offsets, row_src, slot, tile_plan, gate_up_proj.shape[0], K, T)
    if d_out is None:
        d_out = torch.zeros(x.shape, dtype=x.dtype, device=x.device)
    d_out = d_out.to(x.dtype).contiguous()
    d_gu, act_w, dw = ops.gemm_down_backward_fused(d_out, plan, down_proj, gate_up, w)
    if d_w is not None:
        dw = dw + d_w.float()
    d_logits = ops.router_softmax_topk_backward(probs, idx, dw, d_probs, renormalize,
                                                torch.bfloat16)
    d_x = x.new_empty(0)
    join = None
    if need_x:
        d_xs = ops.gemm_gate_up_backward_dx(d_gu, plan, gate_up_proj)
        d_x, join = _gather_backward_beside(
            d_xs, plan, ops.router_linear_backward_dx(d_logits, w_router))
        del d_xs
    d_w2 = _dw_down(d_out, act_w, plan, down_proj, need_w2, acc_w2)
    del act_w
    d_w1 = _dw_gate_up(d_gu, x, plan, gate_up_proj, need_w1, acc_w1)
    d_wr = w_router.new_empty(0)
    if need_wr:
        d_wr = ops.router_linear_backward_dw(d_logits, x)
    if join is not None:
        join()
    return d_x, d_wr, d_w1, d_w2


@moe_layer_bwd.register_fake
def _(d_out, d_probs, d_w, x, w_router, gate_up_proj, down_proj, gate_up, probs, w, idx, counts,
      offsets, row_src, slot, tile_plan, renormalize, need_x, need_wr, need_w1, need_w2,
      acc_w1, acc_w2):
    return (torch.empty_like(x) if need_x else x.new_empty(0),
            torch.empty_like(w_router) if need_wr else w_router.new_empty(0),
            torch.empty_like(gate_up_proj) if need_w1 and acc_w1 is None
            else gate_up_proj.new_empty(0),
            torch.empty_like(down_proj) if need_w2 and acc_w2 is None
            else down_proj.new_empty(0))


def _layer_setup(ctx, inputs, output):
    x, w_router, gate_up_proj, down_proj, _, renormalize, _, _, _ = inputs
    _, probs, w, idx, gu, counts, offsets, row_src, slot, tile_plan = output
    ctx.set_materialize_grads(False)
    ctx.mark_non_differentiable(idx)
    ctx.save_for_backward(x, w_router, gate_up_proj, down_proj, gu, probs, w, idx, counts,
                          offsets, row_src, slot, tile_plan)
    ctx.renormalize = renormalize
    ctx.main_grads = (_main_grad(gate_up_proj), _main_grad(down_proj))


def _layer_backward(ctx, d_out, d_probs, d_w, *unused):
    need_x, need_wr, need_w1, need_w2 = (bool(n) for n in ctx.needs_input_grad[:4])
    if d_out is None and d_probs is None and d_w is None:
        return (None,) * 9
    acc1, acc2 = ctx.main_grads
    d_x, d_wr, d_w1, d_w2 = torch.ops.moe_amd.moe_layer_bwd(
        d_out, d_probs, d_w, *ctx.saved_tensors, ctx.renormalize, need_x, need_wr, need_w1,
        need_w2, acc1 if need_w1 else None, acc2 if need_w2 else None)
    return (d_x if need_x else None, d_wr if need_wr else None,
            d_w1 if need_w1 and acc1 is None else None,
            d_w2 if need_w2 and acc2 is None else None, None, None, None, None, None)


torch.library.register_autograd(f"{_LIB}::moe_layer_fwd", _layer_backward,
                                setup_context=_layer_setup)
