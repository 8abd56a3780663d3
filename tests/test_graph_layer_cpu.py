"""CPU checks of the graph layer's building blocks, each against an independent answer.

* ULP distance: against a brute-force rank of every finite fp16 / bf16 value.
* Lowering: the expanded graph computes what the compound op computes (torch's own kernel on
  the same input), for logsumexp (keepdim or not) and log_softmax (with and without dtype=),
  fp32 and 16-bit; every emitted node carries the lowering mark.
* Rename ledger: chains resolve to the live end; a missing link or a cycle raises.
* apply on a program with several outputs, one of them the fused value and one a value the
  fusion does not touch: the exported signature follows the rename and the program still
  runs and agrees with the module.
"""
import itertools
import sys
from unittest.mock import patch

import pytest
import torch

import neptune_opt
from neptune_opt.ab import _bounded_names, _name_messages
from neptune_opt.verification import Tolerance, first_difference, ulp_distance
from neptune_recognize import ledger
from neptune_recognize.lowering import MARK, lower_compound

RW = sys.modules["neptune_recognize.rewrite"]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_ulp_distance_matches_a_brute_force_rank(dtype):
    bits = torch.arange(-32768, 32768, dtype=torch.int32).to(torch.int16)
    values = bits.view(dtype)
    finite = torch.isfinite(values)
    values = values[finite]
    # rank of each value among the distinct finite values (+0 and -0 are one value)
    distinct = torch.unique(values.float())
    rank = torch.searchsorted(distinct, values.float())
    g = torch.Generator().manual_seed(0)
    i = torch.randint(0, values.numel(), (20000,), generator=g)
    j = torch.randint(0, values.numel(), (20000,), generator=g)
    want = (rank[i] - rank[j]).abs()
    got = ulp_distance(values[i], values[j])
    assert torch.equal(got.long(), want.long())
    zero, nzero = torch.zeros(1, dtype=dtype), -torch.zeros(1, dtype=dtype)
    assert ulp_distance(zero, nzero).item() == 0
    tiny = torch.tensor([torch.finfo(dtype).tiny], dtype=dtype)
    assert ulp_distance(-tiny, tiny).item() == 2 * ulp_distance(zero, tiny).item()


def test_first_difference_texts_and_ulp_slack():
    a = torch.tensor([1.0, 2.0, float("nan")], dtype=torch.bfloat16)
    b = a.clone()
    assert first_difference(a, b) is None
    b[0] = float("inf")
    assert first_difference(a, b) == "output 0 finite classification differs"
    c = a.clone()
    c[1] = torch.nextafter(torch.tensor(2.0), torch.tensor(3.0)).bfloat16() + 0.25
    tight = Tolerance(0.0, 0.0, None)
    assert first_difference(a, c, tight).startswith("output 0: ")
    assert first_difference(a, c, Tolerance(0.0, 0.0, 64)) is None
    assert "ULP bound" in first_difference(a, c, Tolerance(0.0, 0.0, 1))
    assert first_difference((a,), [a]) == "output pytree structure differs"
    assert first_difference(torch.tensor([1, 2]), torch.tensor([1, 3])) == \
        "output 0 integer/bool values differ"


class _LSE(torch.nn.Module):
    def __init__(self, keepdim):
        super().__init__()
        self.keepdim = keepdim

    def forward(self, x):
        return torch.logsumexp(x, dim=-1, keepdim=self.keepdim)


class _LogSoftmax(torch.nn.Module):
    def __init__(self, dtype=None):
        super().__init__()
        self.dtype = dtype

    def forward(self, x):
        return torch.log_softmax(x, dim=-1, dtype=self.dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("module", [_LSE(True), _LSE(False), _LogSoftmax(), _LogSoftmax(torch.float32)],
                         ids=["lse_keep", "lse", "log_softmax", "log_softmax_f32"])
def test_lowering_reproduces_the_compound_op(module, dtype):
    x = (3 * torch.randn(6, 40, generator=torch.Generator().manual_seed(1))).to(dtype)
    x[2, 7] = float("inf")
    x[4, :] = -float("inf")
    ep = torch.export.export(module.eval(), (x,))
    gm = ep.graph_module
    compound = [n.name for n in gm.graph.nodes if n.op == "call_function"
                and ("logsumexp" in str(n.target) or "log_softmax" in str(n.target))]
    assert len(compound) == 1
    assert lower_compound(gm) == 1
    lowered = [n for n in gm.graph.nodes if n.op == "call_function"]
    assert all(n.meta.get(MARK) == compound[0] for n in lowered
               if n.target is not torch.ops.aten._assert_tensor_metadata.default)
    assert not any("logsumexp" in str(n.target) or "log_softmax" in str(n.target) for n in lowered)
    want = module(x)
    got = ep.module()(x)
    assert got.dtype == want.dtype and got.shape == want.shape
    # NaN/inf classes exactly; values within the dtype's rounding of an fp32 evaluation
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    tol = 1e-6 if want.dtype == torch.float32 else float(torch.finfo(want.dtype).eps)
    torch.testing.assert_close(got, want, rtol=tol, atol=tol, equal_nan=True)


def test_lowering_refuses_other_dims_and_leaves_the_graph():
    class Dim0(torch.nn.Module):
        def forward(self, x):
            return torch.logsumexp(x, dim=0)

    ep = torch.export.export(Dim0(), (torch.randn(4, 5),))
    before = str(ep.graph)
    assert lower_compound(ep.graph_module) == 0
    assert str(ep.graph) == before


def test_ledger_chains_and_failures():
    live = {"c", "z"}
    resolve = ledger.resolver({"a": "b", "b": "c", "x": "y"}, live)
    assert resolve("a") == "c" and resolve("c") == "c"
    with pytest.raises(RuntimeError, match="removed intermediate y"):
        resolve("x")
    with pytest.raises(RuntimeError, match="cyclic"):
        ledger.resolver({"p": "q", "q": "p"}, live)("p")
    gm = torch.fx.GraphModule(torch.nn.Module(), torch.fx.Graph())
    shared = gm.meta
    ledger.record(gm, "a", "b")
    ledger.record(gm, "b", "c")
    assert ledger.entries(gm) == {"a": "b", "b": "c"}
    entries = ledger.entries(gm)
    entries["zz"] = "q"                       # a copy: the ledger is unchanged
    assert "zz" not in ledger.entries(gm) and shared is gm.meta


def test_bounded_names_reads_at_most_one_past_the_limit():
    def endless():
        yield from itertools.cycle(("serial", "split"))

    messages = _name_messages("plans", ("serial", "split"))
    with pytest.raises(ValueError, match="distinct"):
        _bounded_names(endless(), ("serial", "split"), messages)
    assert _bounded_names(("split",), ("serial", "split"), messages) == ("split",)
    with pytest.raises(ValueError, match="finite iterable"):
        _bounded_names("serial", ("serial", "split"), messages)
    with pytest.raises(ValueError, match="finite iterable"):
        _bounded_names(3, ("serial", "split"), messages)


@torch.library.custom_op("neptune_cpu_standin2::lse_keep", mutates_args=())
def _lse_keep(x: torch.Tensor) -> torch.Tensor:
    return torch.logsumexp(x, -1, keepdim=True)


@_lse_keep.register_fake
def _(x):
    return x.new_empty(x.shape[:-1] + (1,))


class _TwoOutputs(torch.nn.Module):
    def forward(self, x):
        m = x.amax(-1, keepdim=True)
        lse = m + torch.log(torch.exp(x - m).sum(-1, keepdim=True))
        return lse, x * 2.0


def test_apply_renames_a_fused_graph_output_and_keeps_the_others():
    x = torch.randn(8, 32, generator=torch.Generator().manual_seed(3))
    model = _TwoOutputs().eval()
    ep = torch.export.export(model, (x,)).run_decompositions()
    outputs_before = [s.arg.name for s in ep.graph_signature.output_specs]
    with patch("neptune_codegen.op_handle", lambda *a, **k: _lse_keep._opoverload), \
            patch.object(RW, "_launch_config", return_value=(1024, 4)):
        report = neptune_opt.apply(ep, verify_with=(model, (x,)))
    assert report.fusions and report.verified, report.summary()
    outputs_after = [s.arg.name for s in ep.graph_signature.output_specs]
    live = {n.name for n in ep.graph.nodes}
    assert outputs_after[1] == outputs_before[1] and set(outputs_after) <= live
    fused = [n for n in ep.graph.nodes if n.target is _lse_keep._opoverload]
    assert len(fused) == 1 and outputs_after[0] == fused[0].name
    got = ep.module()(x)
    want = model(x)
    torch.testing.assert_close(got[0], want[0])
    torch.testing.assert_close(got[1], want[1])
