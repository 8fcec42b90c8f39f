"""Benchmark: MoE layer forward+backward on one MI355X.

A step is one forward+backward of the whole expert layer over one batch of
synthetic inputs already resident in HBM: gating linear (MFMA) -> router
softmax/top-k -> permutation -> grouped GEMM-1 + SwiGLU -> grouped GEMM-2 ->
combine, then the full backward (GEMM-2 dX+dSwiGLU fused with the combine
backward, routing-weight gradient reduction, GEMM-2 dW, GEMM-1 dW, router
backward, gating-linear dW (split-K), GEMM-1 dX, gating-linear dX, gather +
add), every kernel hand-written HIP.  Default
workload: the L (Qwen3-30B-A3B) layer, T=65536, H=2048, E=128, K=8, I=768,
bf16.  The expert weights' gradients: autograd's dense tensors, or (the
global-bank workloads, by default) added in place into the weights'
main_grad; either way the bank's gradient accumulates over the layer calls
of one optimizer step (the config's bank_calls), as in training.

Prints ONE JSON line on stdout (progress goes to stderr).  The line carries
the layer throughput (tokens/s), per-kernel HIP-event timings over the timed
steps, the roofline of the dominant grouped GEMM against the 2.5 PFLOP/s
dense bf16 MFMA peak, a CPU baseline (the oracle restatement of the
reference algorithm timed on the host cores on a bounded token sample), and,
outside the timed steps, the times of the routing consumers (load-balancing
losses, routing statistics, expert-bias update) on the layer's router
output.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

METRIC = ("MoE layer fwd+bwd tokens/sec and grouped-GEMM TFLOP/s (% bf16 MFMA peak), 1 GPU")
PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3  # dense fp32 MFMA (the fp32 XS-standard layer's GEMMs)
PEAK_HBM_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# Algorithmic work per launch of each entry point (cfg, plan rows S).
def gemm_flops(name: str, S: int, H: int, I: int) -> float:
    per = {
        "moe_amd_gemm_gate_up_swiglu": 2.0 * S * H * 2 * I,
        "moe_amd_gemm_down": 2.0 * S * I * H,
        "moe_amd_gemm_down_backward_dx_dswiglu": 2.0 * S * H * I,
        "moe_amd_gemm_down_backward_dw": 2.0 * S * H * I,
        "moe_amd_gemm_down_backward_dx_fused": 2.0 * S * H * I,
        "moe_amd_gemm_down_backward_dw_gathered": 2.0 * S * H * I,
        "moe_amd_gemm_gate_up_backward_dx": 2.0 * S * 2 * I * H,
        "moe_amd_gemm_gate_up_backward_dw": 2.0 * S * 2 * I * H,
    }
    return per.get(name.replace("_accumulate", ""), 0.0)


def hbm_bytes(name: str, cfg, touched: int | None = None) -> float:
    """Algorithmic HBM bytes of a launch: each operand read once (routed rows
    as gathered, S*H), each output written once (b = element size); the
    accumulating dW GEMMs read and write the gradients of the `touched`
    experts (those with routed rows) only."""
    T, H, K, E, S, I = cfg.T, cfg.H, cfg.K, cfg.E, cfg.S, cfg.I
    b = 2 if cfg.dtype == torch.bfloat16 else 4
    w1, w2 = E * 2 * I * H * b, E * H * I * b
    f = (E if touched is None else touched) / E
    per = {
        "moe_amd_combine": S * H * b + S * 8 + T * H * b,
        "moe_amd_combine_backward": T * H * b + 2 * S * H * b + S * 12,
        "moe_amd_gather_backward": S * H * b + S * 4 + T * H * b,
        "moe_amd_gather_backward_add": S * H * b + S * 4 + 2 * T * H * b,
        "moe_amd_permute": S * 8 + S * 4 * 2 + E * 4,
        # x rows, gate_up_proj in; gate_up and act out
        "moe_amd_gemm_gate_up_swiglu": S * H * b + w1 + S * 2 * I * b + S * I * b,
        "moe_amd_gemm_down": S * I * b + w2 + S * H * b,
        # d_out rows, down_proj, gate_up, weights in; d_gate_up, act_w, partials out
        "moe_amd_gemm_down_backward_dx_fused": S * H * b + w2 + 2 * S * 2 * I * b + S * I * b
        + S * 3 * 4,
        "moe_amd_gemm_down_backward_dw_gathered": S * H * b + S * I * b + w2,
        "moe_amd_gemm_gate_up_backward_dx": S * 2 * I * b + w1 + S * H * b,
        "moe_amd_gemm_gate_up_backward_dw": S * 2 * I * b + S * H * b + w1,
        "moe_amd_gemm_down_backward_dw_gathered_accumulate": S * H * b + S * I * b + 2 * f * w2,
        "moe_amd_gemm_gate_up_backward_dw_accumulate": S * 2 * I * b + S * H * b + 2 * f * w1,
    }
    return per.get(name, 0.0)


def cpu_baseline(cfg, tokens: int) -> dict:
    """The oracle (pure-torch CPU restatement of the reference layer) timed
    for one fwd+bwd on `tokens` tokens of the workload: gating linear,
    router, experts forward, experts backward, router backward and the
    gating linear's two gradients.  Only the experts the sample routes to
    are materialised (drawn before the clock starts): an expert no row
    reaches costs the reference nothing either."""
    from oracle import moe_oracle as O

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    c = cfg.scaled(tokens)
    T, H, E, K, I, dt = c.T, c.H, c.E, c.K, c.I, c.dtype
    g = torch.Generator().manual_seed(0)
    x = torch.randn(T, H, generator=g).to(dt)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(dt)
    off = bias = None
    if c.skew:
        off = c.skew * (torch.randperm(E, generator=g).float() + 1.0).pow(-c.zipf_s)
    if c.bias_range:
        bias = (torch.rand(E, generator=g) * 2.0 - 1.0) * c.bias_range
    dout = torch.randn(T, H, generator=g).to(dt)

    def route():
        if c.router == "softmax":
            logits = torch.nn.functional.linear(x, wr)
            return logits, O.softmax_router(logits, K, True, off)
        logits = torch.nn.functional.linear(x.float(), wr.float())
        return logits, O.sigmoid_router(logits, bias, K, True, None, None, None, dt)

    _, (_, _, idx0) = route()
    used = torch.unique(idx0)
    remap = torch.full((E,), -1, dtype=torch.int64)
    remap[used] = torch.arange(len(used))
    w1 = (torch.randn(len(used), 2 * I, H, generator=g) * 0.02).to(dt)
    w2 = (torch.randn(len(used), H, I, generator=g) * 0.02).to(dt)
    def step() -> float:
        t0 = time.perf_counter()
        logits, (probs, w, idx) = route()
        sub = remap[idx]
        out, cache = O.experts_forward(x, sub, w, w1, w2)
        if c.backward:
            dx, dw, dw1, dw2, _ = O.experts_backward(cache, x, w, w1, w2, dout)
            if c.router == "softmax":
                dl = O.softmax_router_backward(probs, idx, dw, None, True, logits.dtype).float()
            else:
                dl = O.sigmoid_router_backward(probs, idx, dw, None, True, None)
            _ = dl @ wr.float(), dl.T @ x.float()
        return time.perf_counter() - t0

    # A run under 15 s (the XS and M configurations) counts as the warm-up
    # of 3 timed runs, whose median is reported; longer ones are timed once.
    first = step()
    times = [step() for _ in range(3)] if first < 15.0 else [first]
    dt_s = sorted(times)[len(times) // 2]
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo")
                     if l.startswith("model name"))
    except Exception:
        model = "unknown"
    part = "the full batch" if tokens == cfg.T else f"a {tokens}-token sample"
    return {"value": tokens / dt_s, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{part} of the {cfg.name} layer (H={H}, E={E}, K={K}, I={I}; "
                      f"{len(used)} experts routed to), 1 {'fwd+bwd' if c.backward else 'fwd'} in "
                      f"{dt_s:.3g} s"
                      f"{' (median of 3 timed runs after a warm-up)' if len(times) > 1 else ''}, "
                      f"{'bf16-emulating fp32' if dt == torch.bfloat16 else 'fp32'} math; "
                      f"CPU: {model}"}


def routing_gating_check(cfg, x, wr, inp) -> dict:
    """Outside the timed steps: how many tokens' top-k sets differ when the
    logits come from the MFMA gating kernel instead of torch's F.linear (the
    reference's gating, which the default bench path uses)."""
    from moe_amd import ops
    if x.dtype != torch.bfloat16:
        return {"tokens": cfg.T, "hip_gating": "not applicable (fp32 layer: torch gating only)"}
    with torch.no_grad():
        sig = cfg.router == "sigmoid"
        lt = ops.torch_gating_linear(x.detach(), wr.detach(), sig)
        lh = ops.router_linear(x.detach(), wr.detach(),
                               torch.float32 if sig else torch.bfloat16)
        ids = []
        for lg in (lt, lh):
            if sig:
                _, _, i = ops.router_sigmoid_topk(lg, inp.expert_bias, cfg.K, True)
            else:
                _, _, i = ops.router_softmax_topk(lg, cfg.K, True, inp.logit_offset)
            ids.append(i.sort(dim=1).values)
        diff = int((ids[0] != ids[1]).any(dim=1).sum())
        logit_diff = int((lt != lh).sum())
    return {"tokens": cfg.T, "hip_gating_tokens_with_other_topk_set": diff,
            "hip_gating_logits_differing": logit_diff}


def routing_vs_torch_topk(cfg, x, wr, inp, gating: str, idx) -> dict:
    """Outside the timed steps: the timed step's routing `idx` against the
    reference's own selection on this device -- torch.softmax(logits, fp32)
    then torch.topk (src/models/modeling_qwen3_moe.py:269-270), or
    torch.sigmoid then torch.topk(scores + expert_bias) (src/models/
    router.py:112-127) -- on the logits of the timed gating source."""
    from moe_amd import library
    sig = cfg.router == "sigmoid"
    with torch.no_grad():
        logits = library.gating_logits(x.detach(), wr.detach(), gating, fp32=sig)
        if sig:
            ref = torch.sigmoid(logits) + inp.expert_bias
        else:
            z = logits if inp.logit_offset is None else logits.float() + inp.logit_offset
            ref = torch.softmax(z, dim=-1, dtype=torch.float32)
        tv, ti = torch.topk(ref, cfg.K, dim=-1)
        set_diff = (idx.sort(dim=1).values != ti.sort(dim=1).values).any(dim=1)
        pos_diff = idx != ti
        unequal = (pos_diff & (ref.gather(1, idx) != tv)).any(dim=1)
        counts_eq = torch.equal(torch.bincount(idx.reshape(-1), minlength=cfg.E),
                                torch.bincount(ti.reshape(-1), minlength=cfg.E))
    return {"reference_selection": "torch.topk on the device, on torch."
                                   + ("sigmoid(logits) + expert_bias" if sig
                                      else "softmax(logits, fp32)"),
            "topk_set_mismatch": int(set_diff.sum()),
            "topk_order_only_differences": int((pos_diff.any(dim=1) & ~set_diff).sum()),
            "order_differences_between_unequal_values": int(unequal.sum()),
            "per_expert_counts_equal": bool(counts_eq)}


def _event_ms(fn, reps: int) -> float:
    """Mean HIP-event time of fn() on torch's current stream (2 warm-up calls)."""
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def dense_compare(reps: int = 10) -> dict:
    """Reference points for the grouped GEMMs: hipBLASLt (torch.matmul, bf16
    NT) against this library's dense MFMA mode (moe_amd_router_linear, the
    same template as the grouped GEMMs without the gather) on the dense
    equivalents of GEMM-1 (N = 2I = 1536, K = H = 2048) and GEMM-2 (N = H =
    2048, K = I = 768) at the L shape, M = 262144 rows (half of S: the dense
    mode's 32-bit offsets need M*K*2 < 2^31), and on two square shapes
    (8192^3, 16384^3: long K, few tiles' prologues and epilogues per FLOP,
    the board's MFMA ceiling with either kernel); the two results compared."""
    from moe_amd import ops
    out = {}
    g = torch.Generator(device="cuda").manual_seed(0)
    for name, (m, n, k) in {"gemm1_shape": (262144, 1536, 2048),
                            "gemm2_shape": (262144, 2048, 768),
                            "square_8192": (8192, 8192, 8192),
                            "square_16384": (16384, 16384, 16384)}.items():
        a = torch.randn(m, k, device="cuda", generator=g).to(torch.bfloat16)
        b = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        fl = 2.0 * m * n * k
        t_blas = _event_ms(lambda: a @ b.t(), reps)
        t_ours = _event_ms(lambda: ops.router_linear(a, b, torch.bfloat16), reps)
        d = (a @ b.t()).float() - ops.router_linear(a, b, torch.bfloat16).float()
        out[name] = {"M": m, "N": n, "K": k,
                     "hipblaslt_ms": round(t_blas, 4),
                     "hipblaslt_tflops": round(fl / t_blas / 1e9, 1),
                     "moe_amd_dense_ms": round(t_ours, 4),
                     "moe_amd_dense_tflops": round(fl / t_ours / 1e9, 1),
                     "max_abs_diff": float(d.abs().max())}
        del a, b, d
    return out


def hbm_reference(nbytes: int = 4 << 30, reps: int = 10) -> dict:
    """Attainable HBM rates with torch's own kernels on this board: a device
    copy (reads and writes nbytes) and a sum (reads nbytes)."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    t_copy = _event_ms(lambda: dst.copy_(src), reps)
    t_sum = _event_ms(lambda: src.sum(), reps)
    return {"bytes": nbytes, "copy_ms": round(t_copy, 4),
            "copy_gbs": round(2 * nbytes / t_copy / 1e6, 1),
            "sum_ms": round(t_sum, 4), "sum_read_gbs": round(nbytes / t_sum / 1e6, 1)}


def copy_calibration(nbytes: int) -> None:
    """A plain copy of known size: reads nbytes, writes nbytes per launch."""
    src = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "launches": 3}), flush=True)


# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE and --pmc
# WRITE_SIZE (one pass each) and scaled by the same counters on a plain copy of
# known size (`--copy-calibration`); the commands and per-counter figures are
# in profiles/gemm_hbm_traffic_L.md and profiles/hbm_traffic_retrofit_XS_global_M.md.
RECORDED_TRAFFIC = {
    "L": {
        "gemm_gate_up_swiglu": 11724022260,
        "gemm_down": 4744795525,
        "gemm_down_backward_dx_fused": 8253627728,
        "gemm_down_backward_dw_gathered": 4596779959,
        "gemm_gate_up_backward_dx": 8668277529,
        "gemm_gate_up_backward_dw": 7097372741,
        "torch_gating_linear": 289691204,
        "router_linear_backward_dx": 290595429,
        "router_linear_backward_dw": 318972910,
        "combine": 2420153756,
        "gather_backward": 2686437232,
    },
    "Retrofit": {
        "gemm_gate_up_swiglu": 4259894233,
        "gemm_down": 2187627238,
        "gemm_down_backward_dx_fused": 2953221848,
        "gemm_down_backward_dw_gathered": 6584539798,
        "gemm_gate_up_backward_dx": 4160436454,
        "gemm_gate_up_backward_dw": 12601085429,
        "gemm_down_backward_dw_gathered_accumulate": 3221565168,
        "gemm_gate_up_backward_dw_accumulate": 5932094247,
        "combine": 605117922,
        "gather_backward": 604582303,
        "router_sigmoid_topk": 236798958,
        "router_sigmoid_topk_backward": 236630583,
    },
    "XS global": {
        "gemm_gate_up_swiglu": 988172263,
        "gemm_down": 485318597,
        "gemm_down_backward_dx_fused": 915755323,
        "gemm_down_backward_dw_gathered": 460877930,
        "gemm_gate_up_backward_dx": 841622096,
        "gemm_gate_up_backward_dw": 765743919,
        "gemm_down_backward_dw_gathered_accumulate": 667508511,
        "gemm_gate_up_backward_dw_accumulate": 1205827387,
        "torch_gating_linear": 40041486,
        "router_linear_backward_dx": 40104928,
        "router_linear_backward_dw": 71518478,
        "combine": 168878452,
        "gather_backward": 201893637,
    },
    "M standard": {
        "gemm_gate_up_swiglu": 5058396448,
        "gemm_down": 2587789420,
        "gemm_down_backward_dx_fused": 3937119063,
        "gemm_down_backward_dw_gathered": 2680022403,
        "gemm_gate_up_backward_dx": 4894430789,
        "gemm_gate_up_backward_dw": 4329990543,
        "torch_gating_linear": 147097438,
        "router_linear_backward_dx": 147560983,
        "router_linear_backward_dw": 176374337,
        "combine": 1210121163,
        "gather_backward": 1343266837,
    },
}


def recorded_traffic(cfg_name: str, kernel: str):
    """Measured HBM bytes per launch of `kernel` at a benchmark workload, else None."""
    for key, table in RECORDED_TRAFFIC.items():
        if cfg_name.startswith(key):
            return table.get(kernel)
    return None


def probs_for_consumers(cfg, x, wr, inp):
    """The layer's router probabilities (or sigmoid scores) at the bench shape."""
    from moe_amd import ops
    with torch.no_grad():
        if cfg.router == "softmax":
            logits = ops.router_linear(x.detach(), wr.detach(), torch.bfloat16)
            probs, _, _ = ops.router_softmax_topk(logits, cfg.K, True, inp.logit_offset)
            return probs
        logits = torch.nn.functional.linear(x.detach().float(), wr.detach().float())
        return torch.sigmoid(logits)


def routing_consumers(cfg, probs, dev, reps: int = 5) -> dict:
    """HIP-event times of the routing consumers on one layer at the bench
    shape: Switch and sequence-wise load-balancing losses (fwd+bwd), routing
    statistics, and the bias update of 48 routers (the depth of
    Qwen3-30B-A3B); achieved GB/s of the [T, E] statistics pass."""
    from moe_amd import balancing as Bal
    from moe_amd import ops
    T, E, K = probs.shape[0], probs.shape[1], cfg.K
    seqs = max(1, T // 8192)
    p = probs.detach().requires_grad_(True)
    routers = torch.nn.Module()
    routers.layers = torch.nn.ModuleList()
    for _ in range(48):
        m = torch.nn.Module()
        m.register_buffer("expert_bias", torch.zeros(E, device=dev))
        m.register_buffer("local_tokens_per_expert",
                          torch.full((E,), float(T * K // E), device=dev))
        routers.layers.append(m)

    def once():
        Bal.load_balancing_loss_func((p,), E, K).backward()
        Bal.seq_load_balancing_loss_func((p,), E, K, batch_size=seqs).backward()
        Bal.compute_routing_stats((p.detach(),), K)
        Bal.update_expert_biases(routers, 1e-3)

    once()
    torch.cuda.synchronize()
    events: list = []
    ops.record_kernel_times(events)
    for _ in range(reps):
        once()
    torch.cuda.synchronize()
    ops.record_kernel_times(None)
    per: dict[str, list[float]] = {}
    for name, s, e in events:
        per.setdefault(name.replace("moe_amd_", ""), []).append(s.elapsed_time(e))
    out = {"shape": {"T": T, "E": E, "K": K, "sequences": seqs, "routers": 48},
           "kernels_ms": {k: round(sum(v) / len(v), 4) for k, v in per.items()}}
    st = out["kernels_ms"].get("topk_stats")
    if st:
        nbytes = T * E * probs.element_size()
        out["topk_stats_gbs"] = round(nbytes / st / 1e6, 1)
        out["topk_stats_frac_hbm"] = round(nbytes / st / 1e6 / PEAK_HBM_GBS, 4)
    return out


def kernel_table(per: dict, cfg, steps: int, peak: float, touched: int):
    """Per-entry-point averages, FLOP/s and GB/s from recorded HIP events."""
    kernels = {}
    gemm_ms = gemm_fl = 0.0
    for name, ts in per.items():
        avg = sum(ts) / len(ts)
        fl = gemm_flops(name, cfg.S, cfg.H, cfg.I)
        by = hbm_bytes(name, cfg, touched)
        k = {"launches_per_step": len(ts) / steps, "avg_ms": round(avg, 4)}
        if fl:
            k["tflops"] = round(fl / avg / 1e9, 1)
            k["frac_peak"] = round(fl / avg / 1e9 / peak, 4)
            gemm_ms += avg * len(ts) / steps
            gemm_fl += fl * len(ts) / steps
        if by:
            k["gbs"] = round(by / avg / 1e6, 1)
            k["frac_hbm"] = round(by / avg / 1e6 / PEAK_HBM_GBS, 4)
        kernels[name.replace("moe_amd_", "")] = k
    return kernels, gemm_ms, gemm_fl


def main():
    from moe_amd.library import GATINGS

    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="l")
    ap.add_argument("--gating", default="torch", choices=GATINGS,
                    help="source of the router logits: torch's F.linear (the reference's own "
                         "call: bit-identical logits and routing) or the MFMA gating kernel")
    ap.add_argument("--kernel-steps", type=int, default=5,
                    help="steps of the separate per-kernel timing pass after the timed steps")
    ap.add_argument("--cpu-tokens", type=int, default=0,
                    help="CPU-baseline sample (0: the whole batch, or 128 tokens for banks "
                         "over 2 GB)")
    ap.add_argument("--weight-grads", default="auto", choices=("auto", "autograd", "main_grad"),
                    help="expert-weight gradients as autograd's dense tensors, or added in place "
                         "into the weights' main_grad (fused accumulation; experts without rows "
                         "untouched); auto: main_grad for the global-bank workloads, whose bank "
                         "gradient sums bank_calls layer calls per optimizer step")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--reference-points", action="store_true",
                    help="time hipBLASLt against the dense MFMA mode on the GEMMs' dense "
                         "shapes, and torch's copy / sum for attainable HBM rates; no bench")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device-to-device copy of BYTES (three times): the "
                         "known-size kernel that scales the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.reference_points:
        print(json.dumps({"dense_gemm": dense_compare(), "hbm": hbm_reference()}), flush=True)
        return
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU's share of the layer; runs on more than one GPU "
              "(expert-parallel all-to-all) are not part of this build.", file=sys.stderr)
        sys.exit(2)

    from moe_amd import ops
    from moe_amd.configs import CONFIGS, make_inputs
    from moe_amd.layer import moe_layer

    cfg = CONFIGS[args.config]
    dev = torch.device("cuda:0")
    log(f"[bench] config {cfg.name}: T={cfg.T} H={cfg.H} E={cfg.E} K={cfg.K} I={cfg.I} "
        f"gating={args.gating}")
    inp = make_inputs(cfg, seed=0, device=dev)
    log("[bench] inputs drawn (CPU, fixed draw order) and resident on the GPU")
    x = inp.x.clone().requires_grad_(True)
    wr = inp.w_router.clone().requires_grad_(True)
    w1 = inp.gate_up_proj.requires_grad_(True)
    w2 = inp.down_proj.requires_grad_(True)
    backward = cfg.backward
    weight_grads = args.weight_grads
    if weight_grads == "auto":
        weight_grads = ("main_grad" if backward and cfg.bank_calls > 1
                        and cfg.dtype == torch.bfloat16 else "autograd")
    if weight_grads == "main_grad":
        w1.main_grad = torch.zeros_like(w1)
        w2.main_grad = torch.zeros_like(w2)
    calls = [0]

    def step():
        # One layer call of a training step.  The input and the router are
        # the call's own; the expert bank's gradient sums the bank_calls calls
        # of an optimizer step and is reset before every bank_calls-th call
        # (main_grad zeroed; autograd's .grad dropped, so that the first call
        # hands over its dW and the others add theirs, as in training).
        x.grad = wr.grad = None
        if calls[0] % cfg.bank_calls == 0:
            if weight_grads == "main_grad":
                w1.main_grad.zero_()
                w2.main_grad.zero_()
            w1.grad = w2.grad = None
        calls[0] += 1
        out, probs, w, idx = moe_layer(x, wr, w1, w2, cfg.K, router=cfg.router,
                                       logit_offset=inp.logit_offset,
                                       expert_bias=inp.expert_bias, gating=args.gating)
        if backward:
            out.backward(inp.dout)
        return idx

    for i in range(args.warmup):
        step()
        log(f"[bench] warmup {i + 1}/{args.warmup}")
    torch.cuda.synchronize()

    # Timed steps: nothing but the layer (no per-kernel instrumentation);
    # HIP events between steps, on the stream every kernel is launched on
    # (torch's current stream), for the per-step median beside the mean.
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    calls[0] = 0  # the timed steps start an optimizer step (main_grad zeroed first)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    marks[0].record()
    for i in range(args.steps):
        idx = step()
        marks[i + 1].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1000.0 / args.steps
    step_ms = sorted(marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps))
    log(f"[bench] {args.steps} steps: {ms:.3f} ms/step (median {step_ms[len(step_ms) // 2]:.3f})")

    # Separate pass: the same steps with a HIP-event pair around every
    # kernel launch, for the per-kernel table and the roofline (with the
    # recorder installed the layer runs every kernel in order on one stream,
    # so that each launch is timed alone; the timed steps above overlap the
    # gather backward with the weight-gradient GEMMs on a second stream).
    events: list = []
    calls[0] = 0
    ops.record_kernel_times(events)
    torch.cuda.synchronize()
    k0 = time.perf_counter()
    for _ in range(args.kernel_steps):
        step()
    torch.cuda.synchronize()
    k_ms = (time.perf_counter() - k0) * 1000.0 / max(args.kernel_steps, 1)
    ops.record_kernel_times(None)
    per: dict[str, list[float]] = {}
    for name, s_ev, e_ev in events:
        per.setdefault(name, []).append(s_ev.elapsed_time(e_ev))
    peak = PEAK_BF16_TFLOPS if cfg.dtype == torch.bfloat16 else PEAK_FP32_TFLOPS
    touched = int((torch.bincount(idx.reshape(-1), minlength=cfg.E) > 0).sum())
    kernels, gemm_ms, gemm_fl = kernel_table(per, cfg, args.kernel_steps, peak, touched)
    gemms = {n: ts for n, ts in per.items() if gemm_flops(n, cfg.S, cfg.H, cfg.I)}
    dom = max(gemms, key=lambda n: sum(gemms[n]))
    dom_avg = sum(gemms[dom]) / len(gemms[dom])
    dom_fl = gemm_flops(dom, cfg.S, cfg.H, cfg.I)
    dom_by = hbm_bytes(dom, cfg, touched)
    # The dominant GEMM's bound: MFMA when its arithmetic intensity
    # (algorithmic FLOP per algorithmic HBM byte) exceeds the machine balance
    # peak / 8 TB/s, else HBM (the 1792-expert bank's weight gradients).
    if dom_fl / dom_by >= peak * 1e12 / (PEAK_HBM_GBS * 1e9):
        roof = {"bound": "mfma", "achieved": round(dom_fl / dom_avg / 1e9, 1), "peak": peak,
                "unit": "TFLOP/s"}
    else:
        roof = {"bound": "hbm", "achieved": round(dom_by / dom_avg / 1e6, 1),
                "peak": PEAK_HBM_GBS, "unit": "GB/s"}
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    counts = torch.bincount(idx.reshape(-1), minlength=cfg.E)
    imbalance = counts.max().item() / (cfg.S / cfg.E)
    log(f"[bench] per-kernel pass: {args.kernel_steps} steps, {k_ms:.3f} ms/step")

    result = {
        "metric": METRIC,
        "value": round(cfg.T / (ms / 1000.0), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "step_ms_events": {"median": round(step_ms[len(step_ms) // 2], 4),
                           "min": round(step_ms[0], 4), "max": round(step_ms[-1], 4)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if cfg.dtype == torch.bfloat16 else "fp32",
        "data": "synthetic (seeded N(0,1) inputs, N(0,0.02) random-init weights, drawn on the "
                "CPU in a fixed order, per expert)",
        "config": {"workload": f"{cfg.name} MoE layer {'fwd+bwd' if backward else 'fwd'}",
                   "T": cfg.T, "H": cfg.H, "E": cfg.E, "K": cfg.K, "I": cfg.I,
                   "router": cfg.router, "gating": args.gating,
                   "weight_grads": weight_grads if backward else None,
                   "bank_calls": cfg.bank_calls,
                   "experts_with_rows": touched,
                   "load_imbalance_max_over_mean": round(imbalance, 3)},
        "gemm": {"flops_per_step": gemm_fl, "ms_per_step": round(gemm_ms, 4),
                 "tflops": round(gemm_fl / gemm_ms / 1e9, 1),
                 "frac_peak": round(gemm_fl / gemm_ms / 1e9 / peak, 4),
                 "timed_in": f"separate per-kernel pass of {args.kernel_steps} steps "
                             f"({k_ms:.3f} ms/step with the events)"},
        "roofline": dict(roof, kernel=dom.replace("moe_amd_", ""),
                         algorithmic_bytes=dom_by, flops=dom_fl,
                         traffic=recorded_traffic(cfg.name, dom.replace("moe_amd_", ""))),
        "kernels": kernels,
        "routing": dict(routing_gating_check(cfg, x, wr, inp),
                        timed_gating=args.gating,
                        timed_logits="torch F.linear: bit-identical to the reference's"
                        if args.gating == "torch" else "MFMA gating kernel",
                        timed_step_vs_reference=routing_vs_torch_topk(cfg, x, wr, inp,
                                                                      args.gating, idx)),
    }
    if cfg.router == "softmax" and cfg.backward:
        result["routing_consumers"] = routing_consumers(cfg, probs_for_consumers(cfg, x, wr, inp),
                                                        dev)
    if not args.no_cpu_baseline:
        big = cfg.E * 3 * cfg.H * cfg.I * 2 > 2 * 2**30
        tokens = args.cpu_tokens or (128 if big else cfg.T)
        log(f"[bench] CPU baseline on {tokens} tokens ...")
        result["cpu_baseline"] = cpu_baseline(cfg, tokens)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
