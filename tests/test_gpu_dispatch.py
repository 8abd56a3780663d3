"""GPU tests of the C++ dispatcher kernels (launch-plan replay) of the fold operators.

The first call per input layout runs the operator's Python body and records its launches;
later calls replay them from C++.  Each test checks the replayed result bit for bit against
the Python body's own result on the same input (same kernels, same arguments), the oracle on
the values, and the counters that say which path ran.
"""
import pytest
import torch

import neptune_codegen as CG
from neptune_codegen import dispatch, torch_op
from oracle import references as R

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda:0")


def _qualname(overload):
    return overload._schema.name


def _delta(name, before):
    now = dispatch.stats(name)
    return {k: now[k] - before[k] for k in now}


def test_fold_replay_matches_python_body_and_oracle():
    dev = _dev()
    op = torch_op.op_handle("logsumexp")
    name = _qualname(op)
    g = torch.Generator().manual_seed(3)
    x = (3 * torch.randn(513, 1000, generator=g)).float()
    y = (3 * torch.randn(513, 1000, generator=g)).float()
    xd, yd = x.to(dev), y.to(dev)
    before = dispatch.stats(name)
    first = op(xd)
    second = op(yd)
    third = op(xd)
    torch.cuda.synchronize()
    d = _delta(name, before)
    print("lse stats delta", d, flush=True)
    assert d["replays"] >= 2 and d["python_calls"] <= 1
    assert torch.equal(first, third)
    torch.testing.assert_close(second.cpu(), R.reference("logsumexp", y), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(CG.run("logsumexp", yd), second, rtol=0, atol=0)


def test_split_plan_replays_scratch_buffers():
    dev = _dev()
    op = torch_op.op_handle("logsumexp", plan="split")
    name = _qualname(op)
    g = torch.Generator().manual_seed(4)
    xs = [(4 * torch.randn(24, 9000, generator=g)).bfloat16() for _ in range(3)]
    before = dispatch.stats(name)
    outs = [op(x.to(dev)) for x in xs]
    torch.cuda.synchronize()
    d = _delta(name, before)
    print("split stats delta", d, flush=True)
    assert d["replays"] >= 2
    for x, got in zip(xs, outs):
        want = R.reference("logsumexp", x)
        torch.testing.assert_close(got.cpu().float(), want.to(torch.bfloat16).float(),
                                   rtol=1.6e-2, atol=1e-3)
    assert torch.equal(outs[0], CG.run("logsumexp", xs[0].to(dev), plan="split"))


def test_copying_layout_keeps_the_python_body():
    dev = _dev()
    op = torch_op.op_handle("logsumexp")
    name = _qualname(op)
    g = torch.Generator().manual_seed(5)
    base = torch.randn(6, 40, 128, generator=g).to(dev)
    x = base.permute(1, 0, 2)          # flattening the leading dims needs a copy
    before = dispatch.stats(name)
    a = op(x)
    b = op(x)
    torch.cuda.synchronize()
    d = _delta(name, before)
    print("copy-layout stats delta", d, flush=True)
    assert d["replays"] == 0 and d["python_calls"] == 2
    assert torch.equal(a, b)
    torch.testing.assert_close(a.cpu(), torch.logsumexp(x.cpu(), -1), rtol=1e-5, atol=1e-6)


def test_rms_norm_replay_and_aliased_inputs():
    dev = _dev()
    op = torch_op.state_op_handle("rms_norm", {"eps": 1e-6})
    name = _qualname(op)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(300, 2048, generator=g).bfloat16()
    gamma = (1 + 0.1 * torch.randn(2048, generator=g)).bfloat16()
    xd, gd = x.to(dev), gamma.to(dev)
    before = dispatch.stats(name)
    a = op(xd, gd)
    b = op(xd, gd)
    torch.cuda.synchronize()
    d = _delta(name, before)
    print("rms stats delta", d, flush=True)
    assert d["replays"] >= 1
    assert torch.equal(a, b)
    want = R.rms_norm_reference(x, gamma, 1e-6).float()
    torch.testing.assert_close(a.cpu().float(), want, rtol=1.6e-2, atol=1e-3)
    # gamma aliasing x's first row: never replayed, still correct
    before = dispatch.stats(name)
    c = op(xd, xd[0])
    torch.cuda.synchronize()
    assert _delta(name, before)["replays"] == 0
    want = R.rms_norm_reference(x, x[0], 1e-6).float()
    torch.testing.assert_close(c.cpu().float(), want, rtol=1.6e-2, atol=1e-3)


def test_errors_and_grad_behaviour_unchanged():
    dev = _dev()
    op = torch_op.op_handle("logsumexp")
    with pytest.raises(TypeError):
        op(torch.ones(4, 8, dtype=torch.int32, device=dev))
    x = torch.randn(16, 64, device=dev, requires_grad=True)
    out = op(x)
    assert out.requires_grad
    with pytest.raises(RuntimeError):
        out.sum().backward()
    with torch.no_grad():
        torch.testing.assert_close(op(x), out.detach(), rtol=0, atol=0)


def test_replay_on_side_stream_and_in_graph():
    dev = _dev()
    op = torch_op.op_handle("logsumexp")
    g = torch.Generator().manual_seed(7)
    x = (2 * torch.randn(1024, 512, generator=g)).to(dev)
    want = op(x)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        got = op(x)
    torch.cuda.current_stream().wait_stream(side)
    assert torch.equal(got, want)
    graph = torch.cuda.CUDAGraph()
    static_x = x.clone()
    with torch.cuda.graph(graph):
        static_out = op(static_x)
    for k in range(3):
        static_x.copy_(x * (k + 1))
        graph.replay()
        torch.cuda.synchronize()
        eager = op(x * (k + 1))
        torch.cuda.synchronize()
        assert torch.equal(static_out, eager), f"graph replay {k} differs"
