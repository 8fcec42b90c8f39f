"""The layer captured in a HIP graph: one fwd+bwd of moe_layer (gating
linear, router, permutation, grouped GEMMs, combine, every backward kernel
including the gather backward's second stream) recorded once with
torch.cuda.graph and replayed several times, with other eager work and
synchronisations between the replays; every replay must give the same bits
as the eager call on the same inputs."""
from __future__ import annotations

import pytest
import torch

import moe_amd  # noqa: F401
from moe_amd.experts import experts_forward
from moe_amd.layer import moe_layer

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skip(reason="capturing the layer with torch.cuda.graph ended the process with a "
                            "segmentation fault in the end of the capture (no GPU fault); the "
                            "cause is not established, and the library now refuses capture"),
]
DEV = "cuda"


def _inputs(T, H, E, K, I, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    wr = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(torch.bfloat16)
    dout = torch.randn(T, H, generator=g).to(torch.bfloat16)
    return [t.to(DEV) for t in (x, wr, w1, w2, dout)]


def _layer_step(x, wr, w1, w2, dout, K, gating):
    out, probs, w, idx = moe_layer(x, wr, w1, w2, K, gating=gating)
    grads = torch.autograd.grad(out, (x, wr, w1, w2), dout)
    return (out, probs, w, idx) + grads


def _experts_step(x, wr, w1, w2, dout, K, gating):
    logits = x.detach().float() @ wr.detach().float().T
    w, idx = torch.softmax(logits, -1).topk(K, dim=-1)
    w = (w / w.sum(-1, keepdim=True)).requires_grad_(True)
    out = experts_forward(x, idx, w, w1, w2)
    grads = torch.autograd.grad(out, (x, w, w1, w2), dout)
    return (out,) + grads


@pytest.mark.parametrize("step,gating", [(_layer_step, "torch"), (_layer_step, "hip"),
                                         (_experts_step, "torch")])
def test_graph_replay_matches_eager(step, gating):
    T, H, E, K, I = 4096, 512, 32, 4, 256
    print(f"graph replay {step.__name__} gating={gating}", flush=True)
    x, wr, w1, w2, dout = _inputs(T, H, E, K, I, seed=21)
    leaves = [t.clone().requires_grad_(True) for t in (x, wr, w1, w2)]
    eager = [t.clone() for t in step(*leaves, dout, K, gating)]
    torch.cuda.synchronize()

    # warm-up on a side stream (allocator and library state), then capture
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step(*leaves, dout, K, gating)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static = step(*leaves, dout, K, gating)

    other = torch.randn(2048, 2048, device=DEV)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(static, eager):
            assert torch.equal(a, b), f"replay {rep} differs from eager"
        # eager work of the program between replays
        other = (other @ other.T).tanh()
        step(*leaves, dout, K, gating)
        torch.cuda.synchronize()
