"""Pins of the numpy fold oracle (oracle/fold.py) -- CPU only.

Checks, each of which a plausible slip in the restatement would fail:
  * the reference's chunk status / seen table for exponential folds (golden, tests/golden);
  * the reference's finalizer special values for every exponential fold (golden);
  * serial left fold, balanced tree and whole-row chunk agree, and the empty state is the
    identity of merge, for every non-two-pass skeleton (reference invariant);
  * the zero-floor case [0, 0.5e-30, 0.5e-30] (reference invariant);
  * closed forms: every skeleton against oracle.references (torch) on random rows, in both plans;
  * the attention fold against softmax(scale q k^T + mask) v in float64.
"""
import json
import math
import pathlib

import numpy as np
import pytest
import torch

from oracle import fold as OF
from oracle import references as R

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _dec(v):
    return {"nan": math.nan, "inf": math.inf, "-inf": -math.inf}.get(v, v) if isinstance(v, str) else v


def test_chunk_status_golden():
    table = json.loads((GOLDEN / "lse_chunk_status.json").read_text())
    p = OF.params_for("logsumexp")
    for case in table["cases"]:
        data = [_dec(v) for v in case["data"]]
        states = [OF.chunk("logsumexp", [x], p, 2) for x in data]
        m, acc, seen, status = OF.merge("logsumexp", states[0], states[1], p)
        assert (seen, status) == (case["seen"], case["status"]), case
        assert not np.isnan(acc), "merge must sanitise before transporting"


def test_finalizer_special_values_golden():
    table = json.loads((GOLDEN / "lse_finalizer_cases.json").read_text())
    for case in table["cases"]:
        name = case["skeleton"]
        data = np.array([_dec(v) for v in case["data"]], np.float32)
        got = float(OF.fold_row(name, data, block=1, plan="split"))
        want = _dec(case["expected"])
        if math.isnan(want):
            assert math.isnan(got), case
        elif math.isinf(want):
            assert got == want, case
        else:
            assert math.isclose(got, want, rel_tol=2e-6, abs_tol=1e-6), (case, got)


@pytest.mark.parametrize("name", sorted(n for n, s in OF.SPECS.items() if not s.get("two_pass")))
def test_partition_tree_and_identity(name):
    inv = json.loads((GOLDEN / "merge_invariants.json").read_text())
    data = np.array(inv["partition_data"], np.float32)
    p = OF.params_for(name)
    n = data.size
    b = inv["partition_block"]
    states = [OF.chunk(name, data[i:i + b], p, n) for i in range(0, n, b)]
    left = states[0]
    for s in states[1:]:
        left = OF.merge(name, left, s, p)
    balanced = OF.merge(name, OF.merge(name, states[0], states[1], p), OF.merge(name, states[2], states[3], p), p)
    whole = OF.chunk(name, data, p, n)
    np.testing.assert_allclose(left[:2], whole[:2], rtol=inv["rtol"], atol=inv["atol"])
    np.testing.assert_allclose(balanced[:2], whole[:2], rtol=inv["rtol"], atol=inv["atol"])
    empty = (np.float32(0), np.float32(0), 0, 0)
    np.testing.assert_allclose(OF.merge(name, empty, left, p)[:2], left[:2])
    np.testing.assert_allclose(OF.merge(name, left, empty, p)[:2], left[:2])


def test_zero_floor_case():
    inv = json.loads((GOLDEN / "merge_invariants.json").read_text())
    data = np.array(inv["zero_floor_data"], np.float32)
    for name in inv["zero_floor_skeletons"]:
        p = OF.params_for(name)
        states = [OF.chunk(name, data[i:i + 1], p, 3) for i in range(3)]
        merged = OF.merge(name, OF.merge(name, states[0], states[1], p), states[2], p)
        np.testing.assert_allclose(merged[:2], OF.chunk(name, data, p, 3)[:2], rtol=2e-6, atol=0)


@pytest.mark.parametrize("name", sorted(OF.SPECS))
@pytest.mark.parametrize("plan", ["serial", "split"])
def test_closed_forms(name, plan):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(6, 300, generator=g)
    if name in ("stable_l2", "sumsq_div", "linear_attn", "decay_renorm"):
        x = x.abs() + 0.05
    params = {"eps": 1e-6} if name == "rmsnorm_max" else {}
    got = OF.fold(name, x.numpy(), block=64, plan=plan, **params)
    want = R.reference(name, x, **params).numpy()
    np.testing.assert_allclose(got, want, rtol=R.summation_tolerance(torch.float32, 300), atol=1e-6)


def test_defaults_match_the_reference_declarations():
    """The oracle's parameter defaults and the product registry's `param_defaults` both equal
    the defaults the reference declares per skeleton (golden transcribed from
    neptune_codegen/library.py:19-177 with skeleton.py:255-267's 1.0 fallback)."""
    import json
    import pathlib

    import neptune_codegen as CG

    golden = json.loads((pathlib.Path(__file__).parent / "golden" / "param_defaults.json").read_text())
    declared = golden["defaults"]
    assert set(declared) == set(CG.supported()) == set(OF.SPECS)
    for name, values in declared.items():
        assert CG.param_defaults(name) == values, name
        for arg, value in values.items():
            assert OF.DEFAULTS[arg] == value, (name, arg)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_fold_matches_closed_form(causal):
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(2, 3, 70, 16, generator=g, dtype=torch.float64) for _ in range(3))
    o, lse = OF.attention_fold(q.numpy(), k.numpy(), v.numpy(), causal=causal, block=16)
    s = (q @ k.transpose(-1, -2)) / 4.0
    if causal:
        s = s.masked_fill(~torch.ones(70, 70, dtype=torch.bool).tril(0), float("-inf"))
    np.testing.assert_allclose(o, (torch.softmax(s, -1) @ v).numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(lse, torch.logsumexp(s, -1).numpy(), rtol=1e-12, atol=1e-12)
    ref = R.attention_reference(q.float(), k.float(), v.float(), scale=0.25, causal=causal)
    np.testing.assert_allclose(ref.double().numpy(), o, rtol=1e-4, atol=1e-5)


def _skeleton_names():
    from neptune_codegen.skeleton import SKELETONS

    return sorted(SKELETONS)


@pytest.mark.parametrize("name", _skeleton_names())
def test_graph_reference_matches_the_fused_closed_form(name):
    """graph_reference (the decomposed producer-then-consumer form) equals reference (torch's
    fused closed forms: logsumexp, var/std, ...) on rows with mixed signs and a zero row; a
    slip in either decomposition -- a dropped max shift, a wrong divisor, the floor on the
    wrong side -- would show here."""
    g = torch.Generator().manual_seed(41)
    x = torch.randn(9, 300, generator=g) * torch.tensor([0.01, 1.0, 30.0]).repeat(3)[:, None]
    x[4] = 0.0
    x[5, :7] = 80.0
    want = R.reference(name, x)
    got = R.graph_reference(name, x)
    torch.testing.assert_close(got, want, rtol=2e-5, atol=1e-6, equal_nan=True)
