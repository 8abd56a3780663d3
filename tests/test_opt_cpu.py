"""neptune_opt on the CPU: apply's transaction, preview, refusals and the A/B decision rule.

The HIP op handle is replaced by a CPU stand-in op defined in this module (the reference's own
tests use the same device-free pattern, tests/test_neptune_opt.py:1066-1113).  Everything
above the kernel -- recognition, rewrite, signature renaming, verification, publication --
runs for real.
"""
import sys
from unittest.mock import patch

import pytest
import torch

import neptune_opt
from neptune_opt import ab

RW = sys.modules["neptune_recognize.rewrite"]
X = torch.randn(16, 64, generator=torch.Generator().manual_seed(1))


@torch.library.custom_op("neptune_cpu_standin::lse", mutates_args=())
def _lse(x: torch.Tensor) -> torch.Tensor:
    return torch.logsumexp(x, -1)


@_lse.register_fake
def _(x):
    return x.new_empty(x.shape[:-1])


@torch.library.custom_op("neptune_cpu_standin::wrong", mutates_args=())
def _wrong(x: torch.Tensor) -> torch.Tensor:
    return torch.logsumexp(x, -1) + 1.0


@_wrong.register_fake
def _(x):
    return x.new_empty(x.shape[:-1])


def _standin(op):
    return (patch("neptune_codegen.op_handle", lambda *a, **k: op),
            patch.object(RW, "_launch_config", return_value=(1024, 4)))


class Model(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.w = torch.nn.Parameter(torch.randn(64, 32, generator=torch.Generator().manual_seed(2)))

    def forward(self, x):
        return torch.logsumexp(x @ self.w, dim=-1) * 2.0 + 1


def _exported():
    model = Model().eval()
    return model, torch.export.export(model, (X,)).run_decompositions()


def test_apply_fuses_verifies_and_publishes():
    model, ep = _exported()
    a, b = _standin(torch.ops.neptune_cpu_standin.lse.default)
    with a, b:
        eligible, reason = neptune_opt.preview(ep)
        assert [m.skeleton for m in eligible] == ["logsumexp"], reason
        report = neptune_opt.apply(ep, verify_with=(model, (X,)))
    assert report and report.verified and report.graph_changed and report.verification_cases == 1
    assert [f.skeleton for f in report.fusions] == ["logsumexp"]
    assert report.fusions[0].proof_kind == "exact-symbolic-real-algebra"
    assert "verified" in report.summary() and neptune_opt.LAST_REPORT is report
    targets = [str(n.target) for n in ep.graph.nodes if n.op == "call_function"]
    assert "neptune_cpu_standin.lse.default" in targets and "aten.mm.default" in targets
    assert not any("amax" in t or "exp.default" in t for t in targets)
    torch.testing.assert_close(ep.module()(X), model(X))


def test_failed_verification_leaves_the_program_untouched():
    model, ep = _exported()
    before = str(ep.graph)
    a, b = _standin(torch.ops.neptune_cpu_standin.wrong.default)
    with a, b:
        report = neptune_opt.apply(ep, verify_with=(model, (X,)))
    assert not report and report.skipped[0][0] == "verify-failed"
    assert str(ep.graph) == before


def test_unverified_apply_says_so():
    model, ep = _exported()
    a, b = _standin(torch.ops.neptune_cpu_standin.lse.default)
    with a, b:
        report = neptune_opt.apply(ep)
    assert report.graph_changed and not report.verified
    assert "unverified" in report.summary()


@pytest.mark.parametrize("kwargs,needle", [
    ({"capabilities": "rms_norm"}, "capabilities"), ({"capabilities": ("rms_norm", "rms_norm")}, "distinct"),
    ({"max_regions": 0}, "max_regions"), ({"rtol": float("nan")}, "tolerances"),
    ({"max_ulps": -1}, "max_ulps"), ({"plan": "tiled"}, "plan"),
    ({"verification_inputs": [[X]]}, "tuple")])
def test_argument_refusals_are_reported_not_raised(kwargs, needle):
    model, ep = _exported()
    before = str(ep.graph)
    report = neptune_opt.apply(ep, verify_with=(model, (X,)), **kwargs)
    assert report.skipped and report.skipped[0][0] == "rewrite-failed"
    assert needle in report.skipped[0][1]
    assert str(ep.graph) == before


def test_fatal_device_errors_propagate():
    model, ep = _exported()

    def broken(*a, **k):
        raise RuntimeError("HIP error: hipErrorIllegalAddress (an illegal memory access was encountered)")

    with patch("neptune_codegen.op_handle", broken), patch.object(RW, "_launch_config", return_value=(1024, 4)):
        with pytest.raises(ab.FatalCudaError):
            neptune_opt.apply(ep, verify_with=(model, (X,)))


def test_nothing_to_fuse_is_a_report():
    ep = torch.export.export(torch.nn.Linear(4, 4), (torch.randn(2, 4),))
    report = neptune_opt.apply(ep)
    assert not report and report.skipped[0][0] == "no-fusion"


def test_op_library_surface():
    assert neptune_opt.op_parameters("softcap_lse") == ("beta",)
    assert neptune_opt.op_parameters("logsumexp") == ()
    for name in ("logsumexp", "stable_l2", "softcap_lse", "variance"):
        assert callable(getattr(neptune_opt, name)) and name in neptune_opt.__all__
    with pytest.raises(TypeError, match="beta"):
        neptune_opt.softcap_lse(X)
    with pytest.raises(RuntimeError, match="experimental"):
        neptune_opt.backend(None, ())


def test_choose_faster_decision_rule():
    assert ab.choose_faster(1.0, 0.5)[0] is True
    assert ab.choose_faster(1.0, 0.99)[0] is False           # inside the 3% margin
    assert "SLOWER" in ab.choose_faster(1.0, 2.0)[2]
    assert ab.choose_faster(float("nan"), 1.0)[0] is False
    with pytest.raises(ValueError):
        ab.choose_faster(1.0, 1.0, margin=-1)


def test_compile_best_validates_before_touching_a_device():
    for kwargs in ({"plans": ()}, {"plans": ("serial", "tiled")}, {"capabilities": "rms_norm"},
                   {"reps": 0}, {"margin": float("inf")}):
        with pytest.raises(ValueError):
            neptune_opt.compile_best(Model(), (X,), **kwargs)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="GPU"):
            neptune_opt.compile_best(Model(), (X,))


@torch.library.custom_op("neptune_cpu_standin::rms", mutates_args=())
def _rms(x: torch.Tensor, gamma: torch.Tensor) -> torch.Tensor:
    z = x.float()
    return (z * torch.rsqrt(z.pow(2).mean(-1, keepdim=True) + 1e-6)).to(x.dtype) * gamma


@_rms.register_fake
def _(x, gamma):
    return x.new_empty(x.shape)


class LSE(torch.nn.Module):
    def forward(self, x):
        return torch.logsumexp(x, dim=-1)


class UpcastLSE(torch.nn.Module):
    def forward(self, x):
        return torch.logsumexp(x.float(), dim=-1)


class RMS(torch.nn.Module):
    def __init__(self, width):
        super().__init__()
        g = torch.Generator().manual_seed(3)
        self.gamma = torch.nn.Parameter((1 + 0.1 * torch.randn(width, generator=g)).bfloat16(),
                                        requires_grad=False)

    def forward(self, x):
        z = x.to(torch.float32)
        return (z * torch.rsqrt(z.pow(2).mean(-1, keepdim=True) + 1e-6)).to(x.dtype) * self.gamma


def _calls(ep):
    return [n for n in ep.graph_module.graph.nodes if n.op == "call_function"]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_compound_lowering_casts_are_absorbed_into_the_fold(dtype):
    """logsumexp on a 16-bit input lowers to upcast -> fold -> downcast; the rewrite feeds the
    16-bit tensor to the fold directly (one call, no fp32 copy of the input)."""
    x = (3 * torch.randn(16, 64, generator=torch.Generator().manual_seed(4))).to(dtype)
    model = LSE().eval()
    ep = torch.export.export(model, (x,))
    a, b = _standin(_lse._opoverload)
    with a, b:
        report = neptune_opt.apply(ep, verify_with=(model, (x,)), max_ulps=2)
    assert report.fusions and report.verified is True, report.summary()
    calls = _calls(ep)
    assert [n.target for n in calls] == [_lse._opoverload]
    assert calls[0].args[0].op == "placeholder"
    out = ep.module()(x)
    assert out.dtype == dtype and out.shape == (16,)


def test_explicit_upcast_keeps_the_fp32_result():
    x = torch.randn(16, 64, generator=torch.Generator().manual_seed(5)).bfloat16()
    model = UpcastLSE().eval()
    ep = torch.export.export(model, (x,))
    a, b = _standin(_lse._opoverload)
    with a, b:
        report = neptune_opt.apply(ep, verify_with=(model, (x,)))
    assert report.fusions, report.summary()
    targets = [n.target for n in _calls(ep)]
    assert _lse._opoverload in targets and torch.ops.aten.to.dtype in targets
    assert ep.module()(x).dtype == torch.float32


class RoundTripLSE(torch.nn.Module):
    def forward(self, x):
        return torch.logsumexp(x.float(), dim=-1).to(x.dtype)


def test_user_written_cast_pair_is_absorbed_too():
    x = torch.randn(16, 64, generator=torch.Generator().manual_seed(7)).half()
    model = RoundTripLSE().eval()
    ep = torch.export.export(model, (x,))
    a, b = _standin(_lse._opoverload)
    with a, b:
        report = neptune_opt.apply(ep, verify_with=(model, (x,)), max_ulps=2)
    assert report.fusions and report.verified is True, report.summary()
    fused = [n for n in _calls(ep) if n.target is _lse._opoverload]
    assert len(fused) == 1 and fused[0].args[0].op == "placeholder"
    assert ep.module()(x).dtype == torch.float16


def test_metadata_asserts_do_not_keep_a_fused_region_alive():
    """export records a dtype assert on the region-internal `.to(x.dtype)` value; after the
    rewrite neither it nor the region's arithmetic may remain (the input's assert stays)."""
    x = torch.randn(32, 64, generator=torch.Generator().manual_seed(6)).bfloat16()
    model = RMS(64).eval()
    ep = torch.export.export(model, (x,))
    with patch("neptune_codegen.state_op_handle", lambda *a, **k: _rms._opoverload):
        report = neptune_opt.apply(ep, verify_with=(model, (x,)), capabilities=("rms_norm",),
                                   max_ulps=2)
    assert report.fusions and report.verified is True, report.summary()
    targets = [n.target for n in _calls(ep)]
    assert _rms._opoverload in targets
    leftover = [t for t in targets if t not in (_rms._opoverload,
                                                 torch.ops.aten._assert_tensor_metadata.default)]
    assert leftover == [], leftover
    asserts = [n for n in _calls(ep) if n.target is torch.ops.aten._assert_tensor_metadata.default]
    assert all(n.args[0].op == "placeholder" for n in asserts)


@torch.library.custom_op("neptune_cpu_standin::log_softmax_nanrows", mutates_args=())
def _ls_nan(x: torch.Tensor) -> torch.Tensor:
    z = x.float()
    lse = torch.logsumexp(z, -1, keepdim=True)
    return torch.where(lse == float("inf"), float("nan"), z - lse).to(x.dtype)


@_ls_nan.register_fake
def _(x):
    return x.new_empty(x.shape)


@torch.library.custom_op("neptune_cpu_standin::log_softmax_plain", mutates_args=())
def _ls_plain(x: torch.Tensor) -> torch.Tensor:
    z = x.float()
    return (z - torch.logsumexp(z, -1, keepdim=True)).to(x.dtype)


@_ls_plain.register_fake
def _(x):
    return x.new_empty(x.shape)


class LogSoftmax(torch.nn.Module):
    def forward(self, x):
        return torch.log_softmax(x, dim=-1)


class MinusLSE(torch.nn.Module):
    def forward(self, x):
        return x - torch.logsumexp(x, dim=-1, keepdim=True)


def _readout_standin():
    asked = []

    def handle(name, params=None, nan_posinf_rows=True, lib="neptune", **kw):
        asked.append((name, nan_posinf_rows))
        return (_ls_nan if nan_posinf_rows else _ls_plain)._opoverload

    return asked, patch("neptune_codegen.readout_op_handle", handle)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_log_softmax_lowering_fuses_into_one_readout(dtype):
    """log_softmax lowers to the LSE region plus x - lse and a NaN select for +inf rows; the
    rewrite replaces all of it (and a 16-bit input's cast pair) with one readout op."""
    x = (3 * torch.randn(16, 64, generator=torch.Generator().manual_seed(8))).to(dtype)
    x[3, 5] = float("inf")
    model = LogSoftmax().eval()
    ep = torch.export.export(model, (x,))
    asked, readout = _readout_standin()
    a, b = _standin(_lse._opoverload)
    with a, b, readout:
        report = neptune_opt.apply(ep, verify_with=(model, (x,)), experimental_log_softmax=True,
                                   max_ulps=2)
    assert report.fusions and report.verified is True, report.summary()
    assert asked == [("logsumexp", True)]
    calls = _calls(ep)
    assert [n.target for n in calls] == [_ls_nan._opoverload]
    assert calls[0].args[0].op == "placeholder"
    out = ep.module()(x)
    assert out.dtype == dtype and torch.isnan(out[3]).all()


def test_x_minus_lse_fuses_without_the_nan_select():
    x = (3 * torch.randn(16, 64, generator=torch.Generator().manual_seed(9)))
    model = MinusLSE().eval()
    ep = torch.export.export(model, (x,))
    asked, readout = _readout_standin()
    a, b = _standin(_lse._opoverload)
    with a, b, readout:
        report = neptune_opt.apply(ep, verify_with=(model, (x,)))
    assert report.fusions and report.verified is True, report.summary()
    assert asked == [("logsumexp", False)]
    assert [n.target for n in _calls(ep)] == [_ls_plain._opoverload]


@torch.library.custom_op("neptune_cpu_standin::lse_keepdim", mutates_args=())
def _lse_keep(x: torch.Tensor) -> torch.Tensor:
    return torch.logsumexp(x, -1, keepdim=True)


@_lse_keep.register_fake
def _(x):
    return x.new_empty(x.shape[:-1] + (1,))


def test_lse_with_other_users_is_not_turned_into_a_readout():
    class Both(torch.nn.Module):
        def forward(self, x):
            lse = torch.logsumexp(x, dim=-1, keepdim=True)
            return x - lse, lse * 2

    x = torch.randn(16, 64, generator=torch.Generator().manual_seed(10))
    model = Both().eval()
    ep = torch.export.export(model, (x,))
    asked, readout = _readout_standin()
    a, b = _standin(_lse_keep._opoverload)
    with a, b, readout:
        report = neptune_opt.apply(ep, verify_with=(model, (x,)))
    assert report.fusions, report.summary()
    assert asked == []
    assert _lse_keep._opoverload in [n.target for n in _calls(ep)]
