"""The torch.library registrations (moe_amd/library.py) on the CPU: every op
is registered with a functional schema, the fake implementations give the
shapes and dtypes the real ops return, and a function calling the expert
layer and its gradient traces into one FX graph through the fake and autograd
registrations (no graph break, no kernel run) -- the property the reference's
custom-op registration of its grouped GEMM exists for
(transformers/integrations/moe.py:245-257)."""
from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

import moe_amd  # noqa: F401  (registers the ops)
from moe_amd import _lib
from moe_amd.experts import experts_forward

OPS = ["experts_fwd", "experts_bwd", "moe_layer_fwd", "moe_layer_bwd", "router_linear",
       "router_linear_backward", "softmax_topk", "softmax_topk_backward", "sigmoid_topk",
       "sigmoid_topk_backward"]


# The backward ops' optional fused-accumulation buffers (a weight's
# main_grad) are their only mutable arguments; every other op is functional.
ACCUMULATORS = {"experts_bwd": {"acc_w1", "acc_w2"}, "moe_layer_bwd": {"acc_w1", "acc_w2"}}


@pytest.mark.parametrize("name", OPS)
def test_registered_functional(name):
    op = getattr(torch.ops.moe_amd, name).default
    mutable = {a.name for a in op._schema.arguments if a.alias_info and a.alias_info.is_write}
    assert mutable == ACCUMULATORS.get(name, set())
    assert all(not r.alias_info for r in op._schema.returns)


def _inputs(T=96, H=128, E=8, K=2, I=64):
    bf = torch.bfloat16
    return (torch.empty(T, H, dtype=bf), torch.zeros(T, K, dtype=torch.int64),
            torch.empty(T, K), torch.empty(E, 2 * I, H, dtype=bf), torch.empty(E, H, I, dtype=bf))


def test_fake_shapes():
    T, H, E, K, I = 96, 128, 8, 2, 64
    S = T * K
    with FakeTensorMode():
        x, idx, w, w1, w2 = _inputs(T, H, E, K, I)
        out, gu, act, y, counts, offsets, row_src, slot, plan = torch.ops.moe_amd.experts_fwd(
            x, idx, w, w1, w2, True)
        assert out.shape == (T, H) and out.dtype == torch.bfloat16
        assert gu.shape == (S, 2 * I)
        assert act.shape == (0, I) and y.shape == (0, H)  # bf16: the fused backward needs neither
        assert counts.shape == (E,) and offsets.shape == (E + 1,) and row_src.shape == (S,)
        assert slot.shape == (S,) and counts.dtype == torch.int32
        assert plan.dtype == torch.uint8 and plan.shape[0] == _lib.load().moe_amd_tile_plan_size(S, E)
        _, gu0, *_ = torch.ops.moe_amd.experts_fwd(x, idx, w, w1, w2, False)
        assert gu0.shape == (0, 2 * I)
        xf, w1f, w2f = x.float(), w1.float(), w2.float()
        _, guf, actf, yf, *_ = torch.ops.moe_amd.experts_fwd(xf, idx, w, w1f, w2f, True)
        assert guf.shape == (S, 2 * I) and actf.shape == (S, I) and yf.shape == (S, H)
        assert actf.dtype == torch.float32  # fp32 saves act and y for its unfused backward
        dx, dw, dw1, dw2 = torch.ops.moe_amd.experts_bwd(
            out, x, w, w1, w2, gu, act, y, counts, offsets, row_src, slot, plan, True, False,
            True, None, None)
        assert dx.shape == x.shape and dw.shape == w.shape and dw1.numel() == 0
        assert dw2.shape == w2.shape
        # with fused accumulation buffers the weight gradients come back empty
        acc1, acc2 = torch.empty_like(w1), torch.empty_like(w2)
        _, _, dw1, dw2 = torch.ops.moe_amd.experts_bwd(
            out, x, w, w1, w2, gu, act, y, counts, offsets, row_src, slot, plan, True, True,
            True, acc1, acc2)
        assert dw1.numel() == 0 and dw2.numel() == 0
        wr = torch.empty(E, H, dtype=torch.bfloat16)
        res = torch.ops.moe_amd.moe_layer_fwd(x, wr, w1, w2, K, True, None, True, "hip")
        assert [tuple(r.shape) for r in res[:5]] == [(T, H), (T, E), (T, K), (T, K), (S, 2 * I)]
        assert res[1].dtype == torch.float32 and res[3].dtype == torch.int64
        logits = torch.ops.moe_amd.router_linear(x, wr, torch.float32)
        assert logits.shape == (T, E) and logits.dtype == torch.float32
        p, wt, ix = torch.ops.moe_amd.softmax_topk(logits.bfloat16(), K, True, None)
        assert p.dtype == torch.float32 and wt.shape == (T, K) and ix.dtype == torch.int64
        sc, wt, ix, cnt = torch.ops.moe_amd.sigmoid_topk(logits, None, K, True, 0.0, 0, 0,
                                                         torch.bfloat16, True)
        assert sc.shape == (T, E) and wt.dtype == torch.bfloat16 and cnt.shape == (E,)


def test_experts_and_gradient_trace_into_one_graph():
    """make_fx in fake mode runs only the fake and autograd registrations:
    the graph holds the forward op and, through autograd, the backward op."""
    def fwd_bwd(x, idx, w, w1, w2, dout):
        out = experts_forward(x, idx, w, w1, w2)
        return torch.autograd.grad(out, (x, w, w1, w2), dout)

    x, idx, w, w1, w2 = _inputs()
    x, w, w1, w2 = (t.requires_grad_(True) for t in (x, w, w1, w2))
    dout = torch.empty(x.shape, dtype=torch.bfloat16)
    gm = make_fx(fwd_bwd, tracing_mode="fake")(x, idx, w, w1, w2, dout)
    targets = {str(n.target) for n in gm.graph.nodes if n.op == "call_function"}
    assert "moe_amd.experts_fwd.default" in targets
    assert "moe_amd.experts_bwd.default" in targets


def test_ops_refuse_stream_capture(monkeypatch):
    """Under stream capture every C-ABI call raises before reaching the
    library (HIP graph capture is not supported)."""
    from moe_amd import ops

    def no_call(*args):
        raise AssertionError("the library was called under capture")

    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    monkeypatch.setattr(_lib, "call", no_call)
    with pytest.raises(RuntimeError, match="graph capture"):
        ops._call("moe_amd_permute", 0)


def test_ops_run_on_their_tensors_device(monkeypatch):
    """A launching op switches the current device to that of its first GPU
    tensor (and back) when it differs; with the device already current it
    switches nothing."""
    from types import SimpleNamespace

    from moe_amd import ops

    entered = []

    class FakeDevice:
        def __init__(self, idx):
            self.idx = idx

        def __enter__(self):
            entered.append(self.idx)

        def __exit__(self, *exc):
            return False

    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    monkeypatch.setattr(torch.cuda, "device", FakeDevice)
    seen = []
    op = ops.on_tensor_device(lambda *a, **k: seen.append(list(entered)) or "ran")
    on1 = SimpleNamespace(is_cuda=True, device=torch.device("cuda", 1))
    on0 = SimpleNamespace(is_cuda=True, device=torch.device("cuda", 0))
    assert op(3, on1, x=on0) == "ran" and entered == [1]
    assert op(on0, on1) == "ran" and entered == [1]          # device 0 already current
    assert op(torch.zeros(2), k=None) == "ran" and entered == [1]  # no GPU tensor
    assert seen == [[1], [1], [1]]
