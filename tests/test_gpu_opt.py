"""neptune_opt / neptune_recognize end to end on the GPU: exported models are rewritten into
the HIP fold ops, verified against the eager module, and run.

Tolerances: the verification inside apply (rtol 1e-3 / atol 1e-4, the reference's defaults)
plus an explicit comparison here at BASELINE's fp32 rtol 1e-5 / atol 1e-6 where the fused op
computes the same fp32 readout, and bf16 rtol 1.6e-2 / atol 1e-3 for the structured RMS op.
"""
import pytest
import torch

import neptune_opt

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda:0")


def _say(*a):
    print(*a, flush=True)


def _neptune_ops(ep):
    return [str(n.target) for n in ep.graph.nodes
            if n.op == "call_function" and str(n.target).startswith("neptune.")]


class ScalarFolds(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.w = torch.nn.Parameter(torch.randn(256, 512, generator=torch.Generator().manual_seed(3)) / 16)

    def forward(self, x):
        z = x @ self.w
        m = z.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
        l2 = (m * torch.sqrt(((z / m) ** 2).sum(dim=-1, keepdim=True))).squeeze(-1)
        return torch.logsumexp(z, dim=-1) + 0.5, l2, z.var(dim=-1, unbiased=False)


def test_export_rewrites_scalar_folds_into_hip_ops():
    dev = _dev()
    model = ScalarFolds().to(dev).eval()
    x = torch.randn(64, 256, generator=torch.Generator().manual_seed(4)).to(dev)
    _say("neptune_opt.export: scalar folds on the GPU")
    ep = neptune_opt.export(model, (x,))
    report = neptune_opt.LAST_REPORT
    assert report.verified and sorted(f.skeleton for f in report.fusions) == ["logsumexp", "stable_l2", "variance"], report.summary()
    ops = _neptune_ops(ep)
    assert len(ops) == 3, ops
    got, want = ep.module()(x), model(x)
    for g, w in zip(got, want):
        torch.testing.assert_close(g, w, rtol=1e-5, atol=2e-5)


def test_apply_structured_rms_and_segment_on_the_gpu():
    dev = _dev()

    class RMS(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.gamma = torch.nn.Parameter((1 + 0.1 * torch.randn(1024, generator=torch.Generator().manual_seed(5))).bfloat16())

        def forward(self, x):
            z = x.to(torch.float32)
            r = torch.rsqrt(z.pow(2).mean(-1, keepdim=True) + 1e-6)
            return (z * r).to(x.dtype) * self.gamma

    class Seg(torch.nn.Module):
        def forward(self, data, lengths):
            return torch.segment_reduce(data, "mean", lengths=lengths, initial=7.0)

    rms = RMS().to(dev).eval()
    x = torch.randn(128, 1024, generator=torch.Generator().manual_seed(6)).bfloat16().to(dev)
    _say("apply capabilities=rms_norm (bf16)")
    ep = torch.export.export(rms, (x,))
    report = neptune_opt.apply(ep, verify_with=(rms, (x,)), capabilities=("rms_norm",))
    assert report.verified and [f.skeleton for f in report.fusions] == ["rms_norm"], report.summary()
    assert report.fusions[0].kind == "structured"
    torch.testing.assert_close(ep.module()(x).float(), rms(x).float(), rtol=1.6e-2, atol=1e-3)

    seg = Seg().eval()
    lengths = torch.tensor([3, 0, 5, 8, 1], dtype=torch.int64, device=dev)
    data = torch.randn(17, 64, generator=torch.Generator().manual_seed(7)).half().to(dev)
    _say("apply capabilities=segment_pool (fp16)")
    ep = torch.export.export(seg, (data, lengths))
    report = neptune_opt.apply(ep, verify_with=(seg, (data, lengths)), capabilities=("segment_pool",))
    assert report.verified and [f.skeleton for f in report.fusions] == ["segment_mean"], report.summary()
    got, want = ep.module()(data, lengths), seg(data, lengths)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_experimental_log_softmax_lowering_on_the_gpu():
    dev = _dev()

    class LogSoftmax(torch.nn.Module):
        def forward(self, x):
            return torch.log_softmax(x, dim=-1)

    model = LogSoftmax().eval()
    x = (3 * torch.randn(32, 1000, generator=torch.Generator().manual_seed(8))).to(dev)
    _say("apply experimental_log_softmax (fp32)")
    ep = torch.export.export(model, (x,))
    report = neptune_opt.apply(ep, verify_with=(model, (x,)), experimental_log_softmax=True)
    assert report.verified and [f.skeleton for f in report.fusions] == ["logsumexp"], report.summary()
    assert len(_neptune_ops(ep)) == 1
    torch.testing.assert_close(ep.module()(x), model(x), rtol=1e-5, atol=1e-5)


@pytest.mark.timeout(600)
def test_compile_best_packages_measures_and_decides(tmp_path):
    dev = _dev()
    model = ScalarFolds().to(dev).eval()
    x = torch.randn(64, 256, generator=torch.Generator().manual_seed(9)).to(dev)
    _say("compile_best: AOTI baseline and fused packages")
    choice = neptune_opt.compile_best(model, (x,), package_dir=str(tmp_path), reps=5, rounds=3,
                                      verbose=False)
    _say(str(choice))
    assert choice.report.verified and choice.fused_package is not None, choice.reason
    assert all(m["verified"] for m in choice.sample_metrics), choice.sample_metrics
    assert choice.baseline_ms > 0 and choice.fused_ms > 0
    runner = torch._inductor.aoti_load_package(choice.package_path)
    for g, w in zip(runner(x), model(x)):
        torch.testing.assert_close(g, w, rtol=1e-3, atol=1e-4)


BUNDLE_CHILD = r"""
import sys, torch
ops_library, bundle, package, data = sys.argv[1:5]
torch.ops.load_library(ops_library)
defined = torch.ops.neptune_bundle.load(bundle)
assert defined >= 1, defined
import torch._inductor.codecache  # noqa: F401 -- aoti_load_package reads it, a fresh process lacks it
runner = torch._inductor.aoti_load_package(package)
d = torch.load(data, weights_only=True)
got = runner(d["x"].to("cuda:0"))
got = got[0] if isinstance(got, (tuple, list)) else got
torch.cuda.synchronize()
assert torch.equal(got.cpu(), d["want"]), (got.cpu() - d["want"]).abs().max()
leaked = sorted(m for m in sys.modules if m.split(".")[0] in ("neptune_codegen", "neptune_opt", "neptune_recognize"))
assert not leaked, leaked
print("bundle child ok, operators defined:", defined, flush=True)
"""


@pytest.mark.timeout(600)
def test_fused_package_runs_from_a_bundle_without_the_python_package(tmp_path):
    """A fused AOTI package plus a launch-plan bundle run in a fresh process that never imports
    neptune: libneptune_ops defines the operators and replays the bundled plans; the result is
    bit-identical to the exporting process's run of the same package."""
    import subprocess
    import sys

    from neptune_codegen import dispatch

    dev = _dev()

    class Model(torch.nn.Module):
        def forward(self, x):
            return torch.log_softmax(x, dim=-1), torch.logsumexp(x.float(), dim=-1)

    x = (4 * torch.randn(300, 4096, generator=torch.Generator().manual_seed(31))).bfloat16().to(dev)
    model = Model().eval()
    ep = torch.export.export(model, (x,))
    report = neptune_opt.apply(ep, verify_with=(model, (x,)), experimental_log_softmax=True,
                               max_ulps=2)
    _say(report.summary())
    assert report.verified is True and len(report.fusions) == 2
    ops = _neptune_ops(ep)
    _say("fused graph ops:", ops)
    package = str(tmp_path / "fused.pt2")
    torch._inductor.aoti_compile_and_package(ep, package_path=package)
    runner = torch._inductor.aoti_load_package(package)
    want = runner(x)
    torch.cuda.synchronize()
    qualnames = [o.rsplit(".", 1)[0].replace(".", "::", 1) for o in ops]
    bundle = str(tmp_path / "fused.nepb")
    plans = dispatch.export_bundle(bundle, qualnames)
    _say("bundle plans:", plans, "size:", (tmp_path / "fused.nepb").stat().st_size)
    assert plans >= len(qualnames)      # every layout this process ran for these operators
    data = str(tmp_path / "data.pt")
    torch.save({"x": x.cpu(), "want": want[0].cpu()}, data)
    # the package returns both outputs; the child checks the first (the readout)
    proc = subprocess.run([sys.executable, "-c", BUNDLE_CHILD, str(dispatch.OPS_LIBRARY), bundle,
                           package, data], capture_output=True, text=True, timeout=300)
    _say(proc.stdout[-2000:], proc.stderr[-3000:])
    assert proc.returncode == 0 and "bundle child ok" in proc.stdout
