"""Tensor-level wrappers of the HIP kernels (one function per C entry point).

Every function takes device tensors, allocates its outputs (and workspace)
through torch's caching allocator, enqueues the kernel on torch's current
stream and returns.  Nothing synchronises and nothing falls back to a CPU
path: non-CUDA tensors or a missing library raise.
"""
from __future__ import annotations

import functools
from dataclasses import dataclass

import torch

from . import _lib

TILE_SIZES = (64, 128, 256)

# Optional per-launch timing: when a list is installed with
# record_kernel_times(), every entry point brackets its launch with a pair of
# HIP events on the current stream (the stream the kernels run on).
_events: list | None = None


def record_kernel_times(events: list | None) -> None:
    """Install (a list) or remove (None) the per-launch event recorder.
    Entries are (entry_point_name, start_event, end_event)."""
    global _events
    _events = events


def kernel_timing_active() -> bool:
    """True while record_kernel_times() has a recorder installed."""
    return _events is not None


def _timed(name: str, fn, *args):
    if _events is None:
        return fn(*args)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    res = fn(*args)
    end.record()
    _events.append((name, start, end))
    return res


def _device_of(args, kwargs):
    for a in (*args, *kwargs.values()):
        if isinstance(a, RoutingPlan):
            return a.counts.device
        if getattr(a, "is_cuda", False):
            return a.device
    return None


def on_tensor_device(fn):
    """Runs ``fn`` with the current device set to the device of its first GPU
    tensor argument: the library launches on the current device, while torch
    code works on tensors of any device whatever device is current."""
    @functools.wraps(fn)
    def run(*args, **kwargs):
        dev = _device_of(args, kwargs)
        if dev is None or dev.index is None or dev.index == torch.cuda.current_device():
            return fn(*args, **kwargs)
        with torch.cuda.device(dev.index):
            return fn(*args, **kwargs)
    return run


def _call(name: str, *args) -> None:
    if torch.cuda.is_current_stream_capturing():
        # A test that captured the layer's fwd+bwd with torch.cuda.graph
        # ended the process with a segmentation fault inside the end of the
        # capture (no GPU fault); until that is understood, refuse capture.
        raise RuntimeError(f"moe_amd.{name}: HIP graph capture of the moe_amd kernels is not "
                           "supported; run them eagerly")
    _timed(name, _lib.call, name, *args)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dtype_code(dt: torch.dtype) -> int:
    if dt == torch.bfloat16:
        return _lib.DTYPE_BF16
    if dt == torch.float32:
        return _lib.DTYPE_F32
    raise TypeError(f"moe_amd: unsupported dtype {dt}")


def _need_cuda(*ts: torch.Tensor | None) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "moe_amd kernels run on the GPU only; got a tensor on "
                f"{t.device} (there is no CPU fallback)")


def _contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


# ----------------------------------------------------------------- router

@on_tensor_device
def torch_gating_linear(x: torch.Tensor, weight: torch.Tensor, fp32: bool) -> torch.Tensor:
    """The reference's own gating linear, as torch computes it on this device:
    ``F.linear(x, W)`` (bf16 logits, src/models/modeling_qwen3_moe.py:268-270)
    or ``F.linear(x.float(), W.float())`` (src/models/router.py:107-109).
    Routing decided on these logits is the reference's routing bit for bit;
    recorded as ``torch_gating_linear`` by record_kernel_times()."""
    def run(a, b):
        if fp32:
            return torch.nn.functional.linear(a.float(), b.float())
        return torch.nn.functional.linear(a, b)
    return _timed("torch_gating_linear", run, x, weight)


@on_tensor_device
def router_linear(x: torch.Tensor, weight: torch.Tensor,
                  out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """logits [T,E] = x [T,H] . weight [E,H]^T on MFMA (bf16 inputs, fp32
    accumulation), returned in out_dtype (bf16 or fp32)."""
    _need_cuda(x, weight)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("router_linear takes bf16 hidden states and weight")
    x = _contig(x)
    weight = _contig(weight)
    T, H = x.shape
    E = weight.shape[0]
    if weight.shape[1] != H:
        raise ValueError(f"router_linear: weight {tuple(weight.shape)} vs hidden {tuple(x.shape)}")
    logits = torch.empty(T, E, device=x.device, dtype=out_dtype)
    _call("moe_amd_router_linear", x.data_ptr(), weight.data_ptr(), T, E, H, logits.data_ptr(),
          _dtype_code(out_dtype), _stream(x))
    return logits


def router_fused_supported(E: int, top_k: int) -> bool:
    """Shapes of router_linear_softmax_topk (the router's 16-experts-per-lane
    group shapes)."""
    return (64 < E <= 128 and top_k <= 8) or (128 < E <= 256 and top_k <= 16)


@on_tensor_device
def router_linear_softmax_topk(x: torch.Tensor, weight: torch.Tensor, top_k: int,
                               renormalize: bool = True,
                               logit_offset: torch.Tensor | None = None,
                               return_logits: bool = False):
    """The gating linear with the softmax router fused into its epilogue:
    (probs fp32 [T,E], weights fp32 [T,K], index int64 [T,K][, bf16 logits
    [T,E]]), bit-identical to router_linear(x, weight, bf16) followed by
    router_softmax_topk."""
    _need_cuda(x, weight, logit_offset)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("router_linear_softmax_topk takes bf16 hidden states and weight")
    x = _contig(x)
    weight = _contig(weight)
    T, H = x.shape
    E = weight.shape[0]
    if weight.shape[1] != H:
        raise ValueError(f"router_linear_softmax_topk: weight {tuple(weight.shape)} vs hidden "
                         f"{tuple(x.shape)}")
    dev = x.device
    probs = torch.empty(T, E, device=dev, dtype=torch.float32)
    w = torch.empty(T, top_k, device=dev, dtype=torch.float32)
    idx = torch.empty(T, top_k, device=dev, dtype=torch.int64)
    logits = torch.empty(T, E, device=dev, dtype=torch.bfloat16) if return_logits else None
    if logit_offset is not None:
        logit_offset = _contig(logit_offset.to(torch.float32))
    _call("moe_amd_router_linear_softmax_topk", x.data_ptr(), weight.data_ptr(), T, E, H,
          _ptr(logit_offset), int(top_k), int(renormalize), probs.data_ptr(), w.data_ptr(),
          idx.data_ptr(), _ptr(logits), _stream(x))
    return (probs, w, idx, logits) if return_logits else (probs, w, idx)


def router_fused_sigmoid_supported(E: int, top_k: int, num_groups: int | None = None) -> bool:
    """Shapes of router_linear_sigmoid_topk: 8 lanes per token, 8 or 16
    experts per lane, each expert group scored on one lane."""
    return E % 8 == 0 and E <= 128 and top_k <= 8 and (not num_groups or num_groups <= 8)


@on_tensor_device
def router_linear_sigmoid_topk(x: torch.Tensor, weight: torch.Tensor,
                               expert_bias: torch.Tensor | None, top_k: int,
                               renormalize: bool = True, scaling_factor: float | None = None,
                               num_groups: int | None = None, group_topk: int | None = None,
                               weights_dtype: torch.dtype = torch.float32,
                               tokens_per_expert: torch.Tensor | None = None,
                               return_logits: bool = False):
    """The gating linear with the DeepSeek-V3 router fused into its epilogue:
    (scores fp32 [T,E], weights [T,K] in weights_dtype, index int64 [T,K][,
    fp32 logits [T,E]]), bit-identical to router_linear(x, weight, fp32)
    followed by router_sigmoid_topk with the same arguments; with
    ``tokens_per_expert`` the selection counts are added to it."""
    _need_cuda(x, weight, expert_bias, tokens_per_expert)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("router_linear_sigmoid_topk takes bf16 hidden states and weight")
    x = _contig(x)
    weight = _contig(weight)
    T, H = x.shape
    E = weight.shape[0]
    if weight.shape[1] != H:
        raise ValueError(f"router_linear_sigmoid_topk: weight {tuple(weight.shape)} vs hidden "
                         f"{tuple(x.shape)}")
    dev = x.device
    scores = torch.empty(T, E, device=dev, dtype=torch.float32)
    w = torch.empty(T, top_k, device=dev, dtype=weights_dtype)
    idx = torch.empty(T, top_k, device=dev, dtype=torch.int64)
    logits = torch.empty(T, E, device=dev, dtype=torch.float32) if return_logits else None
    if expert_bias is not None:
        expert_bias = _contig(expert_bias.to(torch.float32))
    grouped = num_groups is not None and group_topk is not None
    _call("moe_amd_router_linear_sigmoid_topk", x.data_ptr(), weight.data_ptr(), T, E, H,
          _ptr(expert_bias), int(top_k), int(renormalize), float(scaling_factor or 0.0),
          int(num_groups) if grouped else 0, int(group_topk) if grouped else 0,
          scores.data_ptr(), w.data_ptr(), _dtype_code(weights_dtype), idx.data_ptr(),
          _ptr(tokens_per_expert), _ptr(logits), _stream(x))
    return (scores, w, idx, logits) if return_logits else (scores, w, idx)


@on_tensor_device
def router_linear_backward_dx(d_logits: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """d_x [T,H] = bf16(d_logits [T,E] . weight [E,H]) on MFMA (bf16 inputs)."""
    _need_cuda(d_logits, weight)
    if d_logits.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("router_linear_backward_dx takes bf16 d_logits and weight")
    d_logits = _contig(d_logits)
    weight = _contig(weight)
    T, E = d_logits.shape
    H = weight.shape[1]
    d_x = torch.empty(T, H, device=d_logits.device, dtype=torch.bfloat16)
    _call("moe_amd_router_linear_backward_dx", d_logits.data_ptr(), weight.data_ptr(), T, E, H,
          d_x.data_ptr(), _stream(d_logits))
    return d_x


@on_tensor_device
def router_linear_backward_f32(d_logits: torch.Tensor, x: torch.Tensor, weight: torch.Tensor,
                               need_x: bool = True, need_w: bool = True):
    """(d_x, d_weight) of the fp32 gating linear F.linear(h.float(), W.float())
    for fp32 d_logits [T,E] and bf16 x [T,H], weight [E,H]: fp32-accurate
    products from a two-term bf16 split of d_logits on the MFMA kernels, each
    gradient rounded once to bf16.  A gradient not asked for is an empty
    tensor."""
    _need_cuda(d_logits, x, weight)
    if (d_logits.dtype != torch.float32 or x.dtype != torch.bfloat16
            or weight.dtype != torch.bfloat16):
        raise TypeError("router_linear_backward_f32 takes fp32 d_logits, bf16 x and weight")
    d_logits = _contig(d_logits)
    x = _contig(x)
    weight = _contig(weight)
    T, E = d_logits.shape
    H = x.shape[1]
    if weight.shape != (E, H):
        raise ValueError(f"router_linear_backward_f32: weight {tuple(weight.shape)} vs ({E}, {H})")
    lib = _lib.load()
    nbytes = lib.moe_amd_router_linear_backward_f32_workspace_size(T, E, H)
    ws = torch.empty(max(nbytes, 16), device=x.device, dtype=torch.uint8)
    d_x = (torch.empty(T, H, device=x.device, dtype=torch.bfloat16) if need_x
           else x.new_empty(0))
    d_w = (torch.empty(E, H, device=x.device, dtype=torch.bfloat16) if need_w
           else weight.new_empty(0))
    _call("moe_amd_router_linear_backward_f32", d_logits.data_ptr(), x.data_ptr(),
          weight.data_ptr(), T, E, H, ws.data_ptr(), ws.numel(),
          d_x.data_ptr() if need_x else None, d_w.data_ptr() if need_w else None, _stream(x))
    return d_x, d_w


@on_tensor_device
def router_linear_backward_dw(d_logits: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """d_weight [E,H] = bf16(d_logits [T,E]^T . x [T,H]) on MFMA, split over
    token chunks with fp32 partials."""
    _need_cuda(d_logits, x)
    if d_logits.dtype != torch.bfloat16 or x.dtype != torch.bfloat16:
        raise TypeError("router_linear_backward_dw takes bf16 d_logits and hidden states")
    d_logits = _contig(d_logits)
    x = _contig(x)
    T, E = d_logits.shape
    H = x.shape[1]
    lib = _lib.load()
    nbytes = lib.moe_amd_router_linear_backward_dw_workspace_size(T, E, H)
    ws = torch.empty(max(nbytes, 16), device=x.device, dtype=torch.uint8)
    d_w = torch.empty(E, H, device=x.device, dtype=torch.bfloat16)
    _call("moe_amd_router_linear_backward_dw", d_logits.data_ptr(), x.data_ptr(), T, E, H,
          ws.data_ptr(), ws.numel(), d_w.data_ptr(), _stream(x))
    return d_w


@on_tensor_device
def router_softmax_topk(logits: torch.Tensor, top_k: int, renormalize: bool = True,
                        logit_offset: torch.Tensor | None = None,
                        tokens_per_expert: torch.Tensor | None = None):
    """softmax(logits (+offset)) -> top-k -> renorm.  Returns (probs fp32 [T,E],
    weights fp32 [T,K], index int64 [T,K])."""
    _need_cuda(logits, logit_offset, tokens_per_expert)
    logits = _contig(logits)
    T, E = logits.shape
    dev = logits.device
    probs = torch.empty(T, E, device=dev, dtype=torch.float32)
    w = torch.empty(T, top_k, device=dev, dtype=torch.float32)
    idx = torch.empty(T, top_k, device=dev, dtype=torch.int64)
    if logit_offset is not None:
        logit_offset = _contig(logit_offset.to(torch.float32))
    if tokens_per_expert is not None:
        assert tokens_per_expert.dtype == torch.float32 and tokens_per_expert.is_contiguous()
    _call("moe_amd_router_softmax_topk", logits.data_ptr(), _dtype_code(logits.dtype),
          _ptr(logit_offset), T, E, top_k, int(renormalize), probs.data_ptr(),
          w.data_ptr(), idx.data_ptr(), _ptr(tokens_per_expert), _stream(logits))
    return probs, w, idx


@on_tensor_device
def router_softmax_topk_backward(probs, topk_index, d_weights, d_probs, renormalize: bool,
                                 logits_dtype: torch.dtype):
    _need_cuda(probs, topk_index, d_weights, d_probs)
    T, E = probs.shape
    K = topk_index.shape[1]
    d_weights = _contig(d_weights.to(torch.float32))
    if d_probs is not None:
        d_probs = _contig(d_probs.to(torch.float32))
    d_logits = torch.empty(T, E, device=probs.device, dtype=logits_dtype)
    _call("moe_amd_router_softmax_topk_backward", probs.data_ptr(), topk_index.data_ptr(),
          d_weights.data_ptr(), _ptr(d_probs), T, E, K, int(renormalize),
          d_logits.data_ptr(), _dtype_code(logits_dtype), _stream(probs))
    return d_logits


@on_tensor_device
def router_sigmoid_topk(logits: torch.Tensor, expert_bias: torch.Tensor | None, top_k: int,
                        renormalize: bool = True, scaling_factor: float | None = None,
                        num_groups: int | None = None, group_topk: int | None = None,
                        weights_dtype: torch.dtype = torch.float32,
                        tokens_per_expert: torch.Tensor | None = None):
    """DeepSeek-V3 routing on fp32 logits.  Returns (scores fp32 [T,E],
    weights [T,K] in weights_dtype, index int64 [T,K])."""
    _need_cuda(logits, expert_bias, tokens_per_expert)
    if logits.dtype != torch.float32:
        raise TypeError("router_sigmoid_topk expects fp32 logits (the gating linear runs in fp32)")
    logits = _contig(logits)
    T, E = logits.shape
    dev = logits.device
    scores = torch.empty(T, E, device=dev, dtype=torch.float32)
    w = torch.empty(T, top_k, device=dev, dtype=weights_dtype)
    idx = torch.empty(T, top_k, device=dev, dtype=torch.int64)
    if expert_bias is not None:
        expert_bias = _contig(expert_bias.to(torch.float32))
    grouped = num_groups is not None and group_topk is not None
    _call("moe_amd_router_sigmoid_topk", logits.data_ptr(), _ptr(expert_bias), T, E, top_k,
          int(renormalize), float(scaling_factor or 0.0), int(num_groups) if grouped else 0,
          int(group_topk) if grouped else 0, scores.data_ptr(), w.data_ptr(),
          _dtype_code(weights_dtype), idx.data_ptr(), _ptr(tokens_per_expert),
          _stream(logits))
    return scores, w, idx


@on_tensor_device
def router_sigmoid_topk_scores(scores: torch.Tensor, expert_bias: torch.Tensor | None,
                               top_k: int, renormalize: bool = True,
                               scaling_factor: float | None = None,
                               num_groups: int | None = None, group_topk: int | None = None,
                               weights_dtype: torch.dtype = torch.bfloat16,
                               tokens_per_expert: torch.Tensor | None = None):
    """DeepSeek-V3 routing from given scores (the reference's torch.sigmoid
    of bf16 logits under bf16 autocast, src/models/router.py:107-140): the
    same selection, weights in torch's bf16 arithmetic.  Returns (weights
    [T,K] in weights_dtype, index int64 [T,K])."""
    _need_cuda(scores, expert_bias, tokens_per_expert)
    s32 = _contig(scores.to(torch.float32))
    T, E = s32.shape
    dev = s32.device
    w = torch.empty(T, top_k, device=dev, dtype=weights_dtype)
    idx = torch.empty(T, top_k, device=dev, dtype=torch.int64)
    if expert_bias is not None:
        expert_bias = _contig(expert_bias.to(torch.float32))
    grouped = num_groups is not None and group_topk is not None
    _call("moe_amd_router_sigmoid_topk_scores", s32.data_ptr(), _ptr(expert_bias), T, E, top_k,
          int(renormalize), float(scaling_factor or 0.0), int(num_groups) if grouped else 0,
          int(group_topk) if grouped else 0, w.data_ptr(), _dtype_code(weights_dtype),
          idx.data_ptr(), _ptr(tokens_per_expert), _stream(s32))
    return w, idx


@on_tensor_device
def router_sigmoid_topk_backward(scores, topk_index, d_weights, d_scores, renormalize: bool,
                                 scaling_factor: float | None):
    """d_logits [T,E] fp32 through the gather / renorm / scaling and the
    sigmoid (d scores * (1 - y) * y, y the scores, read as fp32)."""
    _need_cuda(scores, topk_index, d_weights, d_scores)
    scores = _contig(scores.to(torch.float32))
    T, E = scores.shape
    K = topk_index.shape[1]
    d_weights = _contig(d_weights)
    if d_scores is not None:
        d_scores = _contig(d_scores.to(torch.float32))
    d_logits = torch.empty(T, E, device=scores.device, dtype=torch.float32)
    _call("moe_amd_router_sigmoid_topk_backward", scores.data_ptr(), topk_index.data_ptr(),
          d_weights.data_ptr(), _dtype_code(d_weights.dtype), _ptr(d_scores), T, E, K,
          int(renormalize), float(scaling_factor or 0.0), d_logits.data_ptr(),
          _stream(scores))
    return d_logits


# ------------------------------------------------------------ permutation

@dataclass
class RoutingPlan:
    """Device-side routing metadata produced by :func:`permute`.

    counts [E], offsets [E+1] (exclusive; offsets[E] = rows of real experts),
    row_src [S] (sorted row -> flat t*K+k), slot [S] (flat -> sorted row),
    tile_plan (bytes; starts with the int32 row-tile prefixes [3, E+1] for
    BM = 64/128/256, followed by the per-tile {expert, first row, end row}
    tables the grouped GEMMs read)."""
    counts: torch.Tensor
    offsets: torch.Tensor
    row_src: torch.Tensor
    slot: torch.Tensor
    tile_plan: torch.Tensor
    num_experts: int
    top_k: int
    num_tokens: int

    @property
    def num_rows(self) -> int:
        return self.row_src.numel()

    @property
    def tile_starts(self) -> torch.Tensor:
        E = self.num_experts
        return self.tile_plan[: 3 * (E + 1) * 4].view(torch.int32).view(3, E + 1)

    @property
    def row_tile(self) -> torch.Tensor:
        """The index (into TILE_SIZES) of the row-tile height the token-grouped
        GEMMs run with, chosen on the device (a one-element int32 tensor)."""
        E = self.num_experts
        return self.tile_plan[3 * (E + 1) * 4: 3 * (E + 1) * 4 + 4].view(torch.int32)


@on_tensor_device
def permute(topk_index: torch.Tensor, num_experts: int) -> RoutingPlan:
    """Stable counting sort of the routed (token, k) entries by expert."""
    _need_cuda(topk_index)
    if topk_index.dtype != torch.int64:
        topk_index = topk_index.to(torch.int64)
    topk_index = _contig(topk_index)
    T, K = topk_index.shape
    S = T * K
    E = int(num_experts)
    dev = topk_index.device
    lib = _lib.load()
    ws_bytes = int(lib.moe_amd_permute_workspace_size(S, E))
    ws = torch.empty(max(ws_bytes, 256), device=dev, dtype=torch.uint8)
    counts = torch.empty(E, device=dev, dtype=torch.int32)
    offsets = torch.empty(E + 1, device=dev, dtype=torch.int32)
    row_src = torch.empty(S, device=dev, dtype=torch.int32)
    slot = torch.empty(S, device=dev, dtype=torch.int32)
    plan_bytes = int(lib.moe_amd_tile_plan_size(S, E))
    # zeroed so that the bytes the permutation leaves unwritten (alignment
    # padding, tile-table entries past the tile count) are deterministic too
    tile_plan = torch.zeros(plan_bytes, device=dev, dtype=torch.uint8)
    _call("moe_amd_permute", topk_index.data_ptr(), S, E, ws.data_ptr(), ws.numel(),
          counts.data_ptr(), offsets.data_ptr(), row_src.data_ptr(), slot.data_ptr(),
          tile_plan.data_ptr(), plan_bytes, _stream(topk_index))
    return RoutingPlan(counts, offsets, row_src, slot, tile_plan, E, K, T)


# --------------------------------------------------------- grouped GEMMs

@on_tensor_device
def gemm_gate_up_swiglu(x: torch.Tensor, plan: RoutingPlan, gate_up_proj: torch.Tensor,
                        save_gate_up: bool = True):
    """Returns (gate_up [S,2I] or None, act [S,I])."""
    _need_cuda(x, gate_up_proj)
    E, I2, H = gate_up_proj.shape
    I = I2 // 2
    S = plan.num_rows
    act = torch.empty(S, I, device=x.device, dtype=x.dtype)
    gu = torch.empty(S, I2, device=x.device, dtype=x.dtype) if save_gate_up else None
    _call("moe_amd_gemm_gate_up_swiglu", x.data_ptr(), plan.row_src.data_ptr(), plan.top_k,
          plan.offsets.data_ptr(), plan.tile_plan.data_ptr(), gate_up_proj.data_ptr(),
          plan.num_tokens, S, E, H, I, _dtype_code(x.dtype), _ptr(gu), act.data_ptr(),
          _stream(x))
    return gu, act


@on_tensor_device
def gemm_down(act: torch.Tensor, plan: RoutingPlan, down_proj: torch.Tensor) -> torch.Tensor:
    _need_cuda(act, down_proj)
    E, H, I = down_proj.shape
    S = plan.num_rows
    y = torch.empty(S, H, device=act.device, dtype=act.dtype)
    _call("moe_amd_gemm_down", act.data_ptr(), plan.offsets.data_ptr(),
          plan.tile_plan.data_ptr(), down_proj.data_ptr(), S, E, H, I,
          _dtype_code(act.dtype), y.data_ptr(), _stream(act))
    return y


@on_tensor_device
def gemm_down_backward_dx_dswiglu(dy, plan: RoutingPlan, down_proj, gate_up):
    _need_cuda(dy, down_proj, gate_up)
    E, H, I = down_proj.shape
    S = plan.num_rows
    dgu = torch.empty(S, 2 * I, device=dy.device, dtype=dy.dtype)
    _call("moe_amd_gemm_down_backward_dx_dswiglu", dy.data_ptr(), plan.offsets.data_ptr(),
          plan.tile_plan.data_ptr(), down_proj.data_ptr(), gate_up.data_ptr(), S, E, H, I,
          _dtype_code(dy.dtype), dgu.data_ptr(), _stream(dy))
    return dgu


@on_tensor_device
def gemm_down_backward_fused(d_out, plan: RoutingPlan, down_proj, gate_up, topk_weights):
    """Backward of the combine and of GEMM-2 + SwiGLU in one GEMM, without
    materialising d_y = w * d_out[token] ([S,H]): per routed row, g = d_out[t]
    . down_proj[e]; d_gate_up from d_act = w * g; the routing-weight gradient
    <d_out[t], y[r]> = <g, act[r]> (act recomputed from gate_up).  Returns
    (d_gate_up [S,2I], act_w [S,I] = w * act for gemm_down_backward_dw_gathered,
    d_topk_weights [T,K] in topk_weights' dtype)."""
    _need_cuda(d_out, down_proj, gate_up, topk_weights)
    d_out = _contig(d_out)
    topk_weights = _contig(topk_weights)
    E, H, I = down_proj.shape
    S, T, K = plan.num_rows, plan.num_tokens, plan.top_k
    dev, dt = d_out.device, d_out.dtype
    n_part = int(_lib.load().moe_amd_gemm_down_backward_dx_fused_parts(I))
    dgu = torch.empty(S, 2 * I, device=dev, dtype=dt)
    act_w = torch.empty(S, I, device=dev, dtype=dt)
    part = torch.empty(S, n_part, device=dev, dtype=torch.float32)
    dw = torch.empty(T, K, device=dev, dtype=topk_weights.dtype)
    st = _stream(d_out)
    _call("moe_amd_gemm_down_backward_dx_fused", d_out.data_ptr(), plan.row_src.data_ptr(), K,
          plan.offsets.data_ptr(), plan.tile_plan.data_ptr(), down_proj.data_ptr(),
          gate_up.data_ptr(), topk_weights.data_ptr(), _dtype_code(topk_weights.dtype), T, S, E,
          H, I, _dtype_code(dt), dgu.data_ptr(), act_w.data_ptr(), part.data_ptr(), st)
    _call("moe_amd_weight_grad_reduce", part.data_ptr(), n_part, plan.slot.data_ptr(),
          plan.offsets.data_ptr(), T, K, E, dw.data_ptr(), _dtype_code(dw.dtype), st)
    return dgu, act_w, dw


@on_tensor_device
def gemm_down_backward_dw_gathered(d_out, act_w, plan: RoutingPlan, down_proj_shape, out=None,
                                   scheduled: bool = True):
    """d_down_proj[e] = sum over e's rows r of d_out[token(r)]^T act_w[r]
    ([E,H,I]) with d_out rows gathered through row_src; the dW GEMM of
    gemm_down_backward_fused's output.  ``scheduled`` as for
    gemm_down_backward_dw."""
    _need_cuda(d_out, act_w)
    d_out, act_w = _contig(d_out), _contig(act_w)
    E, H, I = down_proj_shape
    _check_out_shape("gemm_down_backward_dw_gathered", down_proj_shape,
                     _dw_shape("gemm_down_backward_dw_gathered", plan, act_w, d_out, False))
    S = plan.num_rows
    dw = _out_or_new(out, (E, H, I), d_out)
    _call("moe_amd_gemm_down_backward_dw_gathered", d_out.data_ptr(), act_w.data_ptr(),
          plan.row_src.data_ptr(), plan.top_k, plan.offsets.data_ptr(),
          plan.tile_plan.data_ptr() if scheduled else None, plan.num_tokens, S, E, H, I,
          _dtype_code(d_out.dtype), dw.data_ptr(), _stream(d_out))
    return dw


def _dw_shape(name: str, plan: RoutingPlan, rows: torch.Tensor, tokens: torch.Tensor,
              rows_first: bool) -> tuple[int, int, int]:
    """The weight shape two dW-GEMM operands imply -- per-row operand
    `rows` [S, n] and token operand `tokens` [T, m]: [E, n, m] (gate_up: n =
    2I, m = H) or, rows_first False, [E, m, n] (down: m = H, n = I) -- after
    checking them against the plan."""
    if rows.dtype != tokens.dtype:
        raise TypeError(f"{name}: operands of dtypes {rows.dtype} and {tokens.dtype}")
    if rows.dim() != 2 or tokens.dim() != 2 or rows.shape[0] != plan.num_rows \
            or tokens.shape[0] != plan.num_tokens:
        raise ValueError(f"{name}: operands of shapes {tuple(rows.shape)} and "
                         f"{tuple(tokens.shape)} do not match the plan's {plan.num_rows} rows "
                         f"and {plan.num_tokens} tokens")
    n, m = rows.shape[1], tokens.shape[1]
    return (plan.num_experts, n, m) if rows_first else (plan.num_experts, m, n)


def _check_out_shape(name: str, shape, expect) -> None:
    if tuple(shape) != tuple(expect):
        raise ValueError(f"{name}: weight shape {tuple(shape)} does not match the operands' "
                         f"{tuple(expect)}")


def _out_or_new(out: torch.Tensor | None, shape, like: torch.Tensor) -> torch.Tensor:
    """A dW GEMM's output: the caller's `out` (contiguous, of `shape`, like's
    dtype and device) or a new tensor."""
    if out is None:
        return torch.empty(shape, device=like.device, dtype=like.dtype)
    if tuple(out.shape) != tuple(shape) or out.dtype != like.dtype or out.device != like.device \
            or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {like.dtype} tensor of shape {tuple(shape)} "
                         f"on {like.device}")
    return out


def _check_accumulator(acc: torch.Tensor, shape, like: torch.Tensor, name: str) -> None:
    if acc.shape != torch.Size(shape) or acc.dtype != torch.bfloat16 or not acc.is_contiguous() \
            or acc.device != like.device:
        raise ValueError(f"{name}: the accumulator must be a contiguous bf16 tensor of shape "
                         f"{tuple(shape)} on {like.device}, got {acc.dtype} "
                         f"{tuple(acc.shape)} on {acc.device}")


@on_tensor_device
def gemm_down_backward_dw_gathered_accumulate(d_out, act_w, plan: RoutingPlan, acc: torch.Tensor):
    """acc [E,H,I] += gemm_down_backward_dw_gathered(d_out, act_w, plan), in
    place, with autograd's bf16 rounding (the GEMM result rounded to bf16,
    then the bf16 add); experts without rows are not touched."""
    _need_cuda(d_out, act_w)
    d_out, act_w = _contig(d_out), _contig(act_w)
    name = "gemm_down_backward_dw_gathered_accumulate"
    E, H, I = _dw_shape(name, plan, act_w, d_out, False)
    _check_accumulator(acc, (E, H, I), d_out, name)
    _call("moe_amd_gemm_down_backward_dw_gathered_accumulate", d_out.data_ptr(),
          act_w.data_ptr(), plan.row_src.data_ptr(), plan.top_k, plan.offsets.data_ptr(),
          plan.tile_plan.data_ptr(), plan.num_tokens, plan.num_rows, E, H, I,
          _dtype_code(d_out.dtype), acc.data_ptr(), _stream(d_out))
    return acc


@on_tensor_device
def gemm_gate_up_backward_dw_accumulate(dgu, x, plan: RoutingPlan, acc: torch.Tensor):
    """acc [E,2I,H] += gemm_gate_up_backward_dw(dgu, x, plan), in place, as
    gemm_down_backward_dw_gathered_accumulate."""
    _need_cuda(dgu, x)
    dgu, x = _contig(dgu), _contig(x)
    name = "gemm_gate_up_backward_dw_accumulate"
    E, I2, H = _dw_shape(name, plan, dgu, x, True)
    _check_accumulator(acc, (E, I2, H), dgu, name)
    _call("moe_amd_gemm_gate_up_backward_dw_accumulate", dgu.data_ptr(), x.data_ptr(),
          plan.row_src.data_ptr(), plan.top_k, plan.offsets.data_ptr(),
          plan.tile_plan.data_ptr(), plan.num_tokens, plan.num_rows, E, H, I2 // 2,
          _dtype_code(dgu.dtype), acc.data_ptr(), _stream(dgu))
    return acc


@on_tensor_device
def gemm_down_backward_dw(dy, act, plan: RoutingPlan, down_proj_shape, out=None,
                          scheduled: bool = True):
    """d_down_proj [E,H,I].  ``scheduled``: claim tiles from the plan's dW
    schedule (balanced under skew); False walks the tiles statically."""
    _need_cuda(dy, act)
    E, H, I = down_proj_shape
    S = plan.num_rows
    if tuple(dy.shape) != (S, H) or tuple(act.shape) != (S, I) or E != plan.num_experts:
        raise ValueError(f"gemm_down_backward_dw: d_y {tuple(dy.shape)} and act "
                         f"{tuple(act.shape)} do not match the weight shape "
                         f"{tuple(down_proj_shape)} and the plan's {S} rows")
    dw = _out_or_new(out, (E, H, I), dy)
    _call("moe_amd_gemm_down_backward_dw", dy.data_ptr(), act.data_ptr(),
          plan.offsets.data_ptr(), plan.tile_plan.data_ptr() if scheduled else None, S, E, H, I,
          _dtype_code(dy.dtype), dw.data_ptr(), _stream(dy))
    return dw


@on_tensor_device
def gemm_gate_up_backward_dx(dgu, plan: RoutingPlan, gate_up_proj):
    _need_cuda(dgu, gate_up_proj)
    E, I2, H = gate_up_proj.shape
    S = plan.num_rows
    dxs = torch.empty(S, H, device=dgu.device, dtype=dgu.dtype)
    _call("moe_amd_gemm_gate_up_backward_dx", dgu.data_ptr(), plan.offsets.data_ptr(),
          plan.tile_plan.data_ptr(), gate_up_proj.data_ptr(), S, E, H, I2 // 2,
          _dtype_code(dgu.dtype), dxs.data_ptr(), _stream(dgu))
    return dxs


@on_tensor_device
def gemm_gate_up_backward_dw(dgu, x, plan: RoutingPlan, gate_up_proj_shape, out=None,
                             scheduled: bool = True):
    """d_gate_up_proj [E,2I,H]; ``scheduled`` as for gemm_down_backward_dw."""
    _need_cuda(dgu, x)
    dgu, x = _contig(dgu), _contig(x)
    E, I2, H = gate_up_proj_shape
    _check_out_shape("gemm_gate_up_backward_dw", gate_up_proj_shape,
                     _dw_shape("gemm_gate_up_backward_dw", plan, dgu, x, True))
    S = plan.num_rows
    dw = _out_or_new(out, (E, I2, H), dgu)
    _call("moe_amd_gemm_gate_up_backward_dw", dgu.data_ptr(), x.data_ptr(),
          plan.row_src.data_ptr(), plan.top_k, plan.offsets.data_ptr(),
          plan.tile_plan.data_ptr() if scheduled else None, plan.num_tokens, S,
          E, H, I2 // 2, _dtype_code(dgu.dtype), dw.data_ptr(), _stream(dgu))
    return dw


# ---------------------------------------------------------------- combine

@on_tensor_device
def combine(y: torch.Tensor, plan: RoutingPlan, topk_weights: torch.Tensor) -> torch.Tensor:
    _need_cuda(y, topk_weights)
    topk_weights = _contig(topk_weights)
    T, K, E = plan.num_tokens, plan.top_k, plan.num_experts
    H = y.shape[1]
    out = torch.empty(T, H, device=y.device, dtype=y.dtype)
    _call("moe_amd_combine", y.data_ptr(), plan.slot.data_ptr(), plan.offsets.data_ptr(),
          topk_weights.data_ptr(), _dtype_code(topk_weights.dtype), T, K, E, H,
          _dtype_code(y.dtype), out.data_ptr(), _stream(y))
    return out


@on_tensor_device
def combine_backward(d_out, y, plan: RoutingPlan, topk_weights):
    _need_cuda(d_out, y, topk_weights)
    d_out = _contig(d_out)
    topk_weights = _contig(topk_weights)
    T, K, E = plan.num_tokens, plan.top_k, plan.num_experts
    H = y.shape[1]
    dy = torch.empty_like(y)
    dw = torch.empty(T, K, device=y.device, dtype=topk_weights.dtype)
    _call("moe_amd_combine_backward", d_out.data_ptr(), y.data_ptr(), plan.slot.data_ptr(),
          plan.offsets.data_ptr(), topk_weights.data_ptr(), _dtype_code(topk_weights.dtype),
          T, K, E, H, _dtype_code(y.dtype), dy.data_ptr(), dw.data_ptr(), _stream(y))
    return dy, dw


@on_tensor_device
def gather_backward(dxs, plan: RoutingPlan, addend: torch.Tensor | None = None) -> torch.Tensor:
    """dx[t] = sum_k dxs[slot[t,k]] (fp32 sum, one rounding); with ``addend``
    [T,H] (same dtype), dx[t] = round(round(sum) + addend[t])."""
    _need_cuda(dxs, addend)
    T, K, E = plan.num_tokens, plan.top_k, plan.num_experts
    H = dxs.shape[1]
    dx = torch.empty(T, H, device=dxs.device, dtype=dxs.dtype)
    if addend is None:
        _call("moe_amd_gather_backward", dxs.data_ptr(), plan.slot.data_ptr(),
              plan.offsets.data_ptr(), T, K, E, H, _dtype_code(dxs.dtype), dx.data_ptr(),
              _stream(dxs))
    else:
        if addend.dtype != dxs.dtype or tuple(addend.shape) != (T, H):
            raise ValueError("gather_backward: addend must be [T,H] in d_xs' dtype")
        addend = _contig(addend)
        _call("moe_amd_gather_backward_add", dxs.data_ptr(), plan.slot.data_ptr(),
              plan.offsets.data_ptr(), addend.data_ptr(), T, K, E, H, _dtype_code(dxs.dtype),
              dx.data_ptr(), _stream(dxs))
    return dx
