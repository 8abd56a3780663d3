"""Recognition on the CPU: which registered fold a decomposed eager form implements.

Case tables: the reference's own positive and negative recognition cases
(tests/test_recognize.py:33-184 of the reference: the eager forms, the expected skeleton, and
the refusals), written here as eager functions.  Recognition is symbolic (no device work), so
these run without a GPU; rewrites in these tests use a CPU stand-in op patched in for the HIP
op handle, which exists only in this test module.
"""
import sys
from unittest.mock import patch

import pytest
import torch
from torch.export import export
from torch.fx.experimental.proxy_tensor import make_fx

import neptune_recognize as NR

RW = sys.modules["neptune_recognize.rewrite"]
X = torch.randn(16, 64, generator=torch.Generator().manual_seed(0))


def d_logsumexp(t):
    m = t.amax(dim=-1, keepdim=True)
    return (torch.log(torch.exp(t - m).sum(dim=-1, keepdim=True)) + m).squeeze(-1)


def d_stable_l2(t):
    m = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
    return (m * torch.sqrt(((t / m) ** 2).sum(dim=-1, keepdim=True))).squeeze(-1)


def d_softcap(t):
    h = torch.tanh(0.5 * t)
    m = h.amax(dim=-1, keepdim=True)
    return (torch.log(torch.exp(h - m).sum(dim=-1, keepdim=True)) + m).squeeze(-1)


def d_sumsq_div(t):
    m = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
    return ((t * t) / m).sum(dim=-1, keepdim=True).squeeze(-1)


def d_linear_attn(t):
    m = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
    return (t / m).sum(dim=-1, keepdim=True).squeeze(-1)


def d_decay_renorm(t):
    m = t.abs().amax(dim=-1, keepdim=True)
    return (t / (m + 2.0)).sum(dim=-1, keepdim=True).squeeze(-1)


def d_lse_biased(t):
    z = t + 1.5
    m = z.amax(dim=-1, keepdim=True)
    return (torch.log(torch.exp(z - m).sum(dim=-1, keepdim=True)) + m).squeeze(-1)


def d_rmsnorm_max(t):
    r = (t * t).mean(dim=-1, keepdim=True)
    return (t / torch.sqrt(r + 1e-6)).amax(dim=-1)


def d_variance(t):
    m = t.mean(dim=-1, keepdim=True)
    return ((t - m) ** 2).mean(dim=-1)


def d_std(t):
    m = t.mean(dim=-1, keepdim=True)
    return (((t - m) ** 2).mean(dim=-1)).sqrt()


def d_variance_keepdim(t):
    m = t.mean(dim=-1, keepdim=True)
    return ((t - m) ** 2).mean(dim=-1, keepdim=True)


def d_batchnorm_like(t):
    m = t.mean(dim=-1, keepdim=True)
    v = ((t - m) ** 2).mean(dim=-1, keepdim=True)
    return (t - m) / (v + 1e-5).sqrt()


CASES = [
    ("logsumexp", d_logsumexp, {"tiny": 0.0}),
    ("stable_l2", d_stable_l2, {}),
    ("softcap_lse", d_softcap, {"beta": 0.5, "tiny": 0.0}),
    ("sumsq_div", d_sumsq_div, {}),
    ("linear_attn", d_linear_attn, {}),
    ("decay_renorm", d_decay_renorm, {"N": 2.0}),
    ("lse_biased", d_lse_biased, {"alpha": 1.5, "tiny": 0.0}),
    ("rmsnorm_max", d_rmsnorm_max, {"eps": 1e-6}),
    ("variance", d_variance, {}),
    ("std", d_std, {}),
    ("variance", d_variance_keepdim, {}),
    ("variance", d_batchnorm_like, {}),
    ("variance", lambda t: t.var(dim=-1, unbiased=False), {}),
    ("std", lambda t: t.std(dim=-1, unbiased=False), {}),
    ("variance", lambda t: torch.var(t, dim=-1, correction=0), {}),
    ("lse_scaled", lambda t: torch.logsumexp(t / 8.0, dim=-1), {"T": 8.0, "tiny": 0.0}),
]


def d_prod(t):
    m = t.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
    return (t / m).prod(dim=-1)


NEGATIVE = [
    ("product consumer (needs a count)", d_prod, "unfamiliar op"),
    ("reduction over dim 0", lambda t: t.sum(dim=0), "last-dimension"),
    ("x.var(-1): unbiased by default", lambda t: t.var(dim=-1), "unbiased"),
    ("x.std(-1): unbiased by default", lambda t: t.std(dim=-1), "unbiased"),
]


class M(torch.nn.Module):
    def __init__(self, fn):
        super().__init__()
        self.fn = fn

    def forward(self, t):
        return self.fn(t)


def _core_aten(fn):
    return export(M(fn).eval(), (X,)).run_decompositions().graph_module


@pytest.mark.parametrize("want,fn,params", CASES, ids=[f"{c[0]}-{i}" for i, c in enumerate(CASES)])
def test_recognition_case(want, fn, params):
    match, reason = NR.recognize(_core_aten(fn))
    assert match is not None, reason
    assert match.skeleton == want
    assert match.params == pytest.approx(params)


@pytest.mark.parametrize("label,fn,why", NEGATIVE, ids=[n[0] for n in NEGATIVE])
def test_recognition_refusal(label, fn, why):
    match, reason = NR.recognize(_core_aten(fn))
    assert match is None, f"{label} matched {match}"
    assert why in reason


def test_regions_inside_a_multi_input_graph():
    """Independent roots with different data boundaries; a GEMM output is an anchor, never
    erased; recognition is read-only."""
    def model(x, y, weight):
        return d_logsumexp(x), d_logsumexp(y @ weight), d_stable_l2(y), d_rmsnorm_max(x)

    x = torch.arange(15, dtype=torch.float32).reshape(3, 5) / 7
    y = torch.arange(12, dtype=torch.float32).reshape(3, 4) / 5 - 1
    w = torch.arange(24, dtype=torch.float32).reshape(4, 6) / 9
    gm = make_fx(model)(x, y, w)
    before = str(gm.graph)
    matches, reason = NR.recognize_regions(gm)
    assert [m.skeleton for m in matches] == ["logsumexp", "logsumexp", "stable_l2", "rmsnorm_max"], reason
    roots = next(n for n in gm.graph.nodes if n.op == "output").args[0]
    assert [m.region_root for m in matches] == list(roots)
    inputs = [n for n in gm.graph.nodes if n.op == "placeholder"]
    assert matches[0].input_node is inputs[0] and matches[3].input_node is inputs[0]
    assert matches[2].input_node is inputs[1] and NR._op(matches[1].input_node) == "mm"
    for m in matches:
        assert NR.region_contract(m) == (False, None)
        assert m.input_node not in m.region_nodes
        assert m.proof_kind == "exact-symbolic-real-algebra"
    assert str(gm.graph) == before


def test_business_clamp_is_a_preserved_boundary_and_rewrite_keeps_it():
    def model(x):
        bounded = x.clamp(min=-0.5, max=0.75)
        return d_logsumexp(bounded), bounded * 3

    x = torch.tensor([[-20., -1., 0., 2., 30.], [5., 4., 3., 2., 1.]])
    gm = make_fx(model)(x)
    matches, reason = NR.recognize_regions(gm)
    assert len(matches) == 1, reason
    clamp = next(n for n in gm.graph.nodes if NR._op(n) == "clamp")
    assert matches[0].input_node is clamp and clamp not in matches[0].region_nodes
    with patch.object(RW, "_launch_config", return_value=(32, 4)), \
            patch("neptune_codegen.op_handle", return_value=d_logsumexp):
        call, refusal = NR.rewrite_match(gm, matches[0])
    assert refusal is None and call.args == (clamp,)
    torch.testing.assert_close(gm(x), model(x))


def test_outer_multiply_stays_outside_the_region():
    """`l2 * 2.0`: the region ends at the readout; the x2 survives the rewrite."""
    def model(x):
        return d_stable_l2(x) * 2.0

    x = torch.randn(4, 9, generator=torch.Generator().manual_seed(2))
    gm = make_fx(model)(x)
    (match,), _ = NR.recognize_regions(gm)
    with patch.object(RW, "_launch_config", return_value=(32, 4)), \
            patch("neptune_codegen.op_handle", return_value=d_stable_l2):
        call, refusal = NR.rewrite_match(gm, match)
    assert refusal is None
    assert any(NR._op(n) == "mul" and n.args[0] is call for n in gm.graph.nodes)
    torch.testing.assert_close(gm(x), model(x))


@pytest.mark.parametrize("dtype,upcast", [(torch.float16, False), (torch.bfloat16, False),
                                        (torch.bfloat16, True)])
def test_low_precision_regions_keep_their_casts(dtype, upcast):
    def model(x):
        z = x.to(torch.float32) if upcast else x
        return d_rmsnorm_max(z).to(dtype)

    x = (torch.arange(15, dtype=torch.float32).reshape(3, 5) / 7).to(dtype)
    gm = make_fx(model)(x)
    (match,), reason = NR.recognize_regions(gm)
    keepdim, refusal = NR.region_contract(match)
    if upcast:
        assert (keepdim, refusal) == (False, None)
        assert NR._op(match.input_node) == "_to_copy"
    else:
        assert keepdim is None and "low-precision intermediate rounding" in refusal
        assert NR.would_rewrite(gm)[0] is False


def test_structured_rms_and_segment_recognition():
    from neptune_recognize.match import recognize_structured_regions

    def rms(x, gamma):
        z = x.to(torch.float32)
        r = torch.rsqrt(z.pow(2).mean(-1, keepdim=True) + 1e-6)
        return (z * r).to(x.dtype) * gamma

    x = torch.randn(4, 8).bfloat16()
    gamma = torch.randn(8).bfloat16()
    gm = make_fx(rms)(x, gamma)
    (match,), reason = recognize_structured_regions(gm, capabilities=("rms_norm",))
    assert match.skeleton == "rms_norm" and match.params == {"eps": 1e-6}
    assert NR.region_contract(match) == (False, None)

    def seg(data, lengths):
        return torch.segment_reduce(data, "mean", lengths=lengths, initial=7.0)

    gm = make_fx(seg)(torch.randn(6, 3), torch.tensor([2, 0, 4]))
    (match,), reason = recognize_structured_regions(gm, capabilities=("segment_pool",))
    assert match.skeleton == "segment_mean"
    assert match.params == {"initial": 7.0, "offsets": False, "unsafe": False}
    empty, why = recognize_structured_regions(gm, capabilities=("rms_norm",))
    assert empty == [] and "no certified structured region" in why


def test_lowering_expands_logsumexp_only_where_it_fuses():
    from neptune_recognize.lowering import lower_compound, lower_if_it_helps

    gm = _core_aten(lambda t: torch.logsumexp(t, dim=-1))
    gm = torch.fx.GraphModule(gm, gm.graph)
    compound = [n for n in gm.graph.nodes if str(n.target) == "aten.logsumexp.default"]
    if not compound:        # this torch decomposes logsumexp itself: lower a hand-built node
        gm = make_fx(lambda t: torch.ops.aten.logsumexp.default(t, [-1], False))(X)
    assert lower_if_it_helps(gm) == 1
    (match,), _ = NR.recognize_regions(gm)
    assert match.skeleton == "logsumexp"
    assert match.region_root.meta.get("neptune_lowering")
    torch.testing.assert_close(gm(X), torch.logsumexp(X, dim=-1))
    # log_softmax expands too (the readout x - LSE with NaN rows stays outside the LSE region)
    gm2 = make_fx(lambda t: torch.ops.aten._log_softmax.default(t, -1, False))(X)
    assert lower_compound(gm2) == 1
    torch.testing.assert_close(gm2(X), torch.log_softmax(X, -1))
    inf_row = X.clone()
    inf_row[0, 3] = float("inf")
    assert torch.isnan(gm2(inf_row)[0]).all() and torch.isnan(torch.log_softmax(inf_row, -1)[0]).all()
