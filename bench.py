"""Benchmark: MoE layer forward+backward on one MI355X.

A step is one forward+backward of the whole expert layer over one batch of
synthetic inputs already resident in HBM: gating linear (MFMA) -> router
softmax/top-k -> permutation -> grouped GEMM-1 + SwiGLU -> grouped GEMM-2 ->
combine, then the full backward (GEMM-2 dX+dSwiGLU fused with the combine
backward, routing-weight gradient reduction, GEMM-2 dW, GEMM-1 dW, router
backward, gating-linear dW (split-K), GEMM-1 dX, gating-linear dX, gather +
add), every kernel hand-written HIP.  Default
workload: the L (Qwen3-30B-A3B) layer, T=65536, H=2048, E=128, K=8, I=768,
bf16.

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
    return per.get(name, 0.0)


def hbm_bytes(name: str, cfg) -> float:
    """Algorithmic HBM bytes of the gather-shaped kernels (b = 2 for bf16)."""
    T, H, K, E, S = cfg.T, cfg.H, cfg.K, cfg.E, cfg.S
    b = 2
    per = {
        "moe_amd_combine": S * H * b + S * 8 + T * H * b,
        "moe_amd_combine_backward": T * H * b + 2 * S * H * b + S * 12,
        "moe_amd_gather_backward": S * H * b + S * 4 + T * H * b,
        "moe_amd_gather_backward_add": S * H * b + S * 4 + 2 * T * H * b,
        "moe_amd_permute": S * 8 + S * 4 * 2 + E * 4,
    }
    return per.get(name, 0.0)


def cpu_baseline(cfg, tokens: int) -> dict:
    """The oracle (pure-torch CPU restatement of the reference layer) timed
    for one fwd+bwd on `tokens` tokens of the same shape."""
    from oracle import moe_oracle as O
    from moe_amd.configs import make_inputs

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    c = cfg.scaled(tokens)
    inp = make_inputs(c, seed=0, device="cpu")
    t0 = time.perf_counter()
    logits = torch.nn.functional.linear(inp.x, inp.w_router)
    probs, w, idx = O.softmax_router(logits, c.K, True, inp.logit_offset)
    out, cache = O.experts_forward(inp.x, idx, w, inp.gate_up_proj, inp.down_proj)
    dx, dw, dw1, dw2, _ = O.experts_backward(cache, inp.x, w, inp.gate_up_proj, inp.down_proj,
                                             inp.dout)
    dl = O.softmax_router_backward(probs, idx, dw, None, True, logits.dtype)
    _ = dl.float() @ inp.w_router.float(), dl.float().T @ inp.x.float()
    dt = time.perf_counter() - t0
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo")
                     if l.startswith("model name"))
    except Exception:
        model = "unknown"
    return {"value": tokens / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{tokens} tokens of the {cfg.name} layer (H={c.H}, E={c.E}, K={c.K}, "
                      f"I={c.I}, bf16-emulating fp32 math), 1 fwd+bwd, {dt:.1f} s; CPU: {model}"}


def copy_calibration(nbytes: int) -> None:
    """A plain copy of known size: reads nbytes, writes nbytes per launch."""
    src = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "launches": 3}), flush=True)


# HBM bytes per launch of the six grouped GEMMs at the L shape, measured with
# rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE (one pass each) and scaled by
# the same counters on a plain copy of known size (`--copy-calibration`); the
# commands and per-counter figures are in profiles/gemm_hbm_traffic_L.md.
RECORDED_TRAFFIC_L = {
    "gemm_gate_up_swiglu": 9255388063,
    "gemm_down": 5037341382,
    "gemm_down_backward_dx_fused": 7960146801,
    "gemm_down_backward_dw_gathered": 4621847096,
    "gemm_gate_up_backward_dx": 8214588646,
    "gemm_gate_up_backward_dw": 6875762976,
    "router_linear": 302451347,
    "router_linear_backward_dx": 289924521,
    "router_linear_backward_dw": 318980091,
}


def recorded_traffic(cfg_name: str, kernel: str):
    """Measured HBM bytes per launch of `kernel` (L shape only), else None."""
    return RECORDED_TRAFFIC_L.get(kernel) if cfg_name.startswith("L") else None


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="l")
    ap.add_argument("--cpu-tokens", type=int, default=16384)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run a plain device-to-device copy of BYTES (three times): the "
                         "known-size kernel that scales the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
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
    log(f"[bench] config {cfg.name}: T={cfg.T} H={cfg.H} E={cfg.E} K={cfg.K} I={cfg.I}")
    inp = make_inputs(cfg, seed=0, device=dev,
                      weight_device=dev if cfg.E * cfg.H * cfg.I > 2**31 else None)
    x = inp.x.clone().requires_grad_(True)
    wr = inp.w_router.clone().requires_grad_(True)
    w1 = inp.gate_up_proj.clone().requires_grad_(True)
    w2 = inp.down_proj.clone().requires_grad_(True)
    params = (x, wr, w1, w2)
    router = cfg.router

    def step():
        for p in params:
            p.grad = None
        out, probs, w, idx = moe_layer(x, wr, w1, w2, cfg.K, router=router,
                                       logit_offset=inp.logit_offset,
                                       expert_bias=inp.expert_bias)
        out.backward(inp.dout)
        return idx

    for i in range(args.warmup):
        step()
        log(f"[bench] warmup {i + 1}/{args.warmup}")
    torch.cuda.synchronize()

    events: list = []
    ops.record_kernel_times(events)
    # HIP events between steps, on the stream every kernel is launched on
    # (torch's current stream), for the per-step median next to the wall-clock mean.
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    marks[0].record()
    for i in range(args.steps):
        idx = step()
        marks[i + 1].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ops.record_kernel_times(None)
    ms = (t1 - t0) * 1000.0 / args.steps
    step_ms = sorted(marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps))
    log(f"[bench] {args.steps} steps: {ms:.3f} ms/step (median {step_ms[len(step_ms) // 2]:.3f})")

    per: dict[str, list[float]] = {}
    for name, s, e in events:
        per.setdefault(name, []).append(s.elapsed_time(e))
    kernels = {}
    gemm_ms = gemm_fl = 0.0
    for name, ts in per.items():
        avg = sum(ts) / len(ts)
        fl = gemm_flops(name, cfg.S, cfg.H, cfg.I)
        by = hbm_bytes(name, cfg)
        k = {"launches_per_step": len(ts) / args.steps, "avg_ms": round(avg, 4)}
        if fl:
            k["tflops"] = round(fl / avg / 1e9, 1)
            k["frac_peak"] = round(fl / avg / 1e9 / PEAK_BF16_TFLOPS, 4)
            gemm_ms += avg * len(ts) / args.steps
            gemm_fl += fl * len(ts) / args.steps
        if by:
            k["gbs"] = round(by / avg / 1e6, 1)
            k["frac_hbm"] = round(by / avg / 1e6 / PEAK_HBM_GBS, 4)
        kernels[name.replace("moe_amd_", "")] = k
    gemms = {n: ts for n, ts in per.items() if gemm_flops(n, cfg.S, cfg.H, cfg.I)}
    dom = max(gemms, key=lambda n: sum(gemms[n]))
    dom_avg = sum(gemms[dom]) / len(gemms[dom])
    dom_fl = gemm_flops(dom, cfg.S, cfg.H, cfg.I)
    achieved = dom_fl / dom_avg / 1e9
    counts = torch.bincount(idx.reshape(-1), minlength=cfg.E)
    imbalance = counts.max().item() / (cfg.S / cfg.E)

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
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs, N(0,0.02) random-init weights)",
        "config": {"workload": f"{cfg.name} MoE layer fwd+bwd", "T": cfg.T, "H": cfg.H,
                   "E": cfg.E, "K": cfg.K, "I": cfg.I, "router": cfg.router,
                   "load_imbalance_max_over_mean": round(imbalance, 3)},
        "gemm": {"flops_per_step": gemm_fl, "ms_per_step": round(gemm_ms, 4),
                 "tflops": round(gemm_fl / gemm_ms / 1e9, 1),
                 "frac_peak": round(gemm_fl / gemm_ms / 1e9 / PEAK_BF16_TFLOPS, 4)},
        "roofline": {"bound": "mfma", "kernel": dom.replace("moe_amd_", ""),
                     "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": recorded_traffic(cfg.name, dom.replace("moe_amd_", ""))},
        "kernels": kernels,
    }
    result["routing_consumers"] = routing_consumers(cfg, probs_for_consumers(cfg, x, wr, inp), dev)
    if not args.no_cpu_baseline:
        log(f"[bench] CPU baseline on {args.cpu_tokens} tokens ...")
        result["cpu_baseline"] = cpu_baseline(cfg, args.cpu_tokens)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
