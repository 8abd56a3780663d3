"""GPU parity of the scalar folds (serial, split, two-pass) against the CPU oracle.

Tolerances are BASELINE.json's: fp32 rtol 1e-5 / atol 1e-6; bf16/fp16 rtol 1.6e-2 / atol 1e-3.
Inputs are generated on the CPU from fixed seeds and copied to the device, so the oracle and
the kernel see identical values.
"""
import math

import pytest
import torch

import neptune_codegen as CG
from oracle import references as R

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-5, 1e-6), torch.bfloat16: (1.6e-2, 1e-3), torch.float16: (1.6e-2, 1e-3)}


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda:0")


def _say(*a):
    print(*a, flush=True)


def _check(name, x_cpu, got, **params):
    """BASELINE tolerance, plus a tight check: within one ulp of the storage dtype of the fp32
    oracle (the kernel accumulates in fp32 and rounds once), which a permuted or dropped
    element would fail even where the BASELINE tolerance would not."""
    want = R.reference(name, x_cpu, **params)
    rtol, atol = TOL[x_cpu.dtype]
    got = got.cpu().float().reshape(want.shape)
    torch.testing.assert_close(got, want.to(x_cpu.dtype).float() if x_cpu.dtype != torch.float32 else want,
                               rtol=rtol, atol=atol)
    if x_cpu.dtype != torch.float32:
        ulp = torch.finfo(x_cpu.dtype).eps
        torch.testing.assert_close(got, want, rtol=ulp, atol=1e-6)


def test_cfg1_logsumexp_fp32_seed0():
    dev = _dev()
    g = torch.Generator().manual_seed(0)
    x = 3 * torch.randn(8192, 1024, generator=g)
    _say("cfg1 logsumexp fp32 [8192,1024]")
    _check("logsumexp", x, CG.run("logsumexp", x.to(dev)))


@pytest.mark.parametrize("width", [128, 1000, 4096, 32000])
def test_cfg2_logsumexp_bf16_widths(width):
    dev = _dev()
    g = torch.Generator().manual_seed(1)
    rows = 16384 if width <= 4096 else 2048
    x = (4 * torch.randn(rows, width, generator=g)).bfloat16()
    _say(f"cfg2 logsumexp bf16 [{rows},{width}]")
    _check("logsumexp", x, CG.run("logsumexp", x.to(dev)))


def test_cfg2_split_bf16():
    dev = _dev()
    g = torch.Generator().manual_seed(2)
    x = (4 * torch.randn(64, 262144, generator=g)).bfloat16()
    _say("cfg2 split logsumexp bf16 [64,262144]")
    _check("logsumexp", x, CG.run("logsumexp", x.to(dev), plan="split"))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", sorted(CG.supported()))
@pytest.mark.parametrize("plan", ["serial", "split"])
def test_every_skeleton_every_dtype(name, dtype, plan):
    dev = _dev()
    sk = CG.SKELETONS[name]
    if plan == "split" and sk.two_pass:
        # a split needs the pair merge, which two-pass folds refuse (their carried state
        # would need the second pass's inputs); the run raises before any launch
        with pytest.raises(NotImplementedError, match="two_pass needs extended carried state"):
            CG.run(name, torch.ones(4, 8, dtype=dtype, device=dev), plan="split", block=256)
        return
    g = torch.Generator().manual_seed(7)
    for rows, width in ((5, 1), (33, 77), (16, 1000), (3, 5000)):
        x = torch.randn(rows, width, generator=g)
        if name in ("stable_l2", "sumsq_div", "linear_attn", "decay_renorm"):
            x = x.abs() + 0.1
        x = x.to(dtype)
        params = {"eps": 1e-6} if name == "rmsnorm_max" else {}
        _say(f"skeleton {name} {dtype} {plan} [{rows},{width}]")
        got = CG.run(name, x.to(dev), plan=plan, block=256 if plan == "split" else None, **params)
        want = R.reference(name, x, **params)
        rtol, atol = TOL[dtype]
        if dtype == torch.float32 and name in ("variance", "std", "sumsq_div", "linear_attn",
                                               "decay_renorm", "stable_l2", "rmsnorm_max"):
            rtol = R.summation_tolerance(dtype, width)
        torch.testing.assert_close(got.cpu().float(), want.to(dtype).float(), rtol=rtol, atol=atol)
        if dtype != torch.float32:
            torch.testing.assert_close(got.cpu().float(), want, rtol=torch.finfo(dtype).eps, atol=1e-5)


@pytest.mark.parametrize("name", ["stable_l2", "linear_attn", "sumsq_div", "decay_renorm",
                                  "rmsnorm_max", "variance"])
def test_quotient_terms_at_extreme_magnitudes(name):
    """Terms divide by a per-tile producer value through one shared reciprocal; rows whose
    magnitudes are denormal (divisor < 2^-126), tiny, or huge must still match the oracle."""
    dev = _dev()
    g = torch.Generator().manual_seed(11)
    params = {"eps": 1e-6} if name == "rmsnorm_max" else {}
    for scale in (1e-39, 1e-30, 3e-20, 1.0, 1e18, 1e30):
        if name == "rmsnorm_max" and scale > 1e19:
            # x^2 overflows: the running mean is inf on both sides of a merge and the repair
            # sqrt(eps + s)/sqrt(eps + s2) is inf/inf = NaN, in the reference's algebra too
            # (its Triton repair is the same ratio); the closed form says 0.
            continue
        x = torch.rand(8, 700, generator=g) + 0.05
        x = (x * scale).float()
        _say(f"quotient fold {name} scale {scale:g}")
        got = CG.run(name, x.to(dev), **params).cpu()
        want = R.reference(name, x, **params)
        ok = torch.isfinite(want)
        assert torch.equal(torch.isfinite(got), ok), (name, scale)
        # results in the denormal range carry fewer significant bits than fp32's 24: there
        # the bound is absolute, one smallest normal
        torch.testing.assert_close(got[ok], want[ok], rtol=R.summation_tolerance(torch.float32, 700),
                                   atol=torch.finfo(torch.float32).tiny)


@pytest.mark.parametrize("name", ["stable_l2", "sumsq_div", "rmsnorm_max"])
def test_repair_slopes_at_extreme_magnitudes_split(name):
    """Repair slopes run through the hardware sqrt / rsq / reciprocal with power-of-two
    rescaling outside [2^-64, 2^64]; the split plan evaluates them at every merge of partial
    states.  rmsnorm_max with eps = 1e-35 (positive, as the split plan requires) at 1e-15 and
    1e-12 puts the slope's sqrt and rsq arguments (the running mean of x^2 plus eps) below
    2^-64 while x^2 stays a normal number."""
    dev = _dev()
    g = torch.Generator().manual_seed(12)
    cases = [(name, {"eps": 1e-35} if name == "rmsnorm_max" else {}, s)
             for s in ((1e-15, 1e-12, 1.0, 1e15) if name == "rmsnorm_max"
                       else (1e-39, 1e-30, 1.0, 1e18, 1e30))]
    for skel, params, scale in cases:
        x = ((torch.rand(6, 3000, generator=g) + 0.05) * scale).float()
        want = R.reference(skel, x, **params)
        for plan, block in (("serial", None), ("split", 256)):
            _say(f"repair slopes {skel} {params} scale {scale:g} plan {plan}")
            got = CG.run(skel, x.to(dev), plan=plan, block=block, **params).cpu()
            ok = torch.isfinite(want)
            assert torch.equal(torch.isfinite(got), ok), (skel, scale, plan)
            torch.testing.assert_close(got[ok], want[ok],
                                       rtol=R.summation_tolerance(torch.float32, 3000),
                                       atol=torch.finfo(torch.float32).tiny)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name", ["rmsnorm_max", "stable_l2", "variance", "softcap_lse"])
def test_wide_rows_at_default_shapes(name, dtype):
    """Widths 8192-32000 at the default launch shapes: 16-bit resident rows of 256-512 lanes,
    one-wave rows with 8 slots per lane, one-row workgroups, several tiles per lane."""
    dev = _dev()
    g = torch.Generator().manual_seed(13)
    params = {"eps": 1e-6} if name == "rmsnorm_max" else {}
    for width in (8192, 16384, 32000):
        x = torch.randn(6, width, generator=g)
        if name == "stable_l2":
            x = x.abs() + 0.1
        x = x.to(dtype)
        _say(f"wide rows {name} {dtype} [6,{width}]")
        got = CG.run(name, x.to(dev), **params)
        want = R.reference(name, x, **params)
        rtol, atol = TOL[dtype]
        if dtype == torch.float32 and name != "softcap_lse":
            rtol = R.summation_tolerance(dtype, width)
        torch.testing.assert_close(got.cpu().float(), want.to(dtype).float(), rtol=rtol, atol=atol)


def test_repeated_calls_reuse_their_launch_and_stay_exact():
    """A repeated serial call reuses the first call's kernel and launch shape: calls that
    differ in alignment, strides, keepdim or a parameter value must not share it."""
    dev = _dev()
    g = torch.Generator().manual_seed(23)
    base = torch.randn(64, 1001, generator=g).bfloat16()
    xd = base.to(dev)
    views = [xd[:, :1000], xd[:, 1:], xd[:, :1000], xd[:, 1:]]   # 16-byte aligned, then not
    for view in views:
        _say(f"repeated call, offset {view.storage_offset()}")
        got = CG.run("logsumexp", view)
        torch.testing.assert_close(got.cpu().float(), R.reference("logsumexp", view.cpu()).bfloat16().float(),
                                   rtol=torch.finfo(torch.bfloat16).eps, atol=1e-5)
    kept = CG.run("logsumexp", views[0], keepdim=True)
    assert kept.shape == (64, 1)
    xs = torch.randn(32, 512, generator=g)
    for beta in (1.0, 2.0, 1.0):
        got = CG.run("softcap_lse", xs.to(dev), beta=beta)
        torch.testing.assert_close(got.cpu(), R.reference("softcap_lse", xs, beta=beta), rtol=1e-5, atol=1e-6)
    # the split plan: the repeated call puts the four partial arrays in one allocation
    xw = torch.randn(3, 40000, generator=g)
    want = R.reference("logsumexp", xw)
    first = CG.run("logsumexp", xw.to(dev), plan="split")
    for _ in range(3):
        again = CG.run("logsumexp", xw.to(dev), plan="split")
        assert torch.equal(again, first)
    torch.testing.assert_close(first.cpu(), want, rtol=1e-5, atol=1e-6)


def test_strided_views_and_keepdim():
    dev = _dev()
    g = torch.Generator().manual_seed(3)
    base = torch.randn(6, 40, 24, generator=g)
    base_dev = base.to(dev)
    views = [lambda b: b[:, :, ::2], lambda b: b.transpose(1, 2), lambda b: b[:, 3, :],
             lambda b: b.transpose(0, 2)[1:], lambda b: b[:, :, 1:]]
    for i, view in enumerate(views):
        v = view(base)
        for keep in (False, True):
            _say(f"strided view {i} keepdim={keep} shape={tuple(v.shape)} stride={v.stride()}")
            got = CG.run("logsumexp", view(base_dev), keepdim=keep)
            want = torch.logsumexp(v, dim=-1, keepdim=keep)
            assert got.shape == want.shape
            torch.testing.assert_close(got.cpu(), want, rtol=1e-5, atol=1e-6)


def test_logsumexp_nonfinite_status_rows():
    dev = _dev()
    inf, nan = float("inf"), float("nan")
    rows = [[nan, inf, 1.0], [inf, -inf, 1.0], [-inf, -inf, -inf], [0.0, -100.0, -200.0],
            [nan, -inf, -inf], [1.0, 2.0, inf], [-inf, 1.0, -inf]]
    for plan in ("serial", "split"):
        for dtype in (torch.float32, torch.bfloat16):
            x = torch.tensor(rows, dtype=dtype)
            # widen each row so the nonfinite values land in different lanes and tiles
            wide = torch.full((len(rows), 3000), -inf, dtype=dtype)
            wide[:, ::1000] = x
            for t in (x, wide):
                _say(f"nonfinite {plan} {dtype} width={t.shape[1]}")
                got = CG.run("logsumexp", t.to(dev), plan=plan, block=256 if plan == "split" else None)
                want = torch.logsumexp(t.float(), dim=-1).to(dtype)
                torch.testing.assert_close(got.cpu(), want, equal_nan=True, rtol=1e-5, atol=1e-6)


def test_empty_rows_and_rank1():
    dev = _dev()
    assert CG.run("logsumexp", torch.empty(0, 8, device=dev)).shape == (0,)
    x = torch.randn(9)
    got = CG.run("logsumexp", x.to(dev))
    assert got.shape == ()
    assert math.isclose(float(got), float(torch.logsumexp(x, 0)), rel_tol=1e-5)


def test_custom_op_registration_runs_hip():
    dev = _dev()
    op = CG.op_handle("lse_scaled", params={"T": 3.0})
    x = torch.randn(4, 300)
    got = op(x.to(dev))
    torch.testing.assert_close(got.cpu(), torch.logsumexp(x / 3.0, -1), rtol=1e-5, atol=1e-6)


def test_split_back_to_back_calls_and_graph_replays():
    """Split-plan calls of different shapes back to back (several virtual rows per workgroup
    when nparts is small), and several replays of a captured graph with eager calls in
    between: each result must match the oracle (no state leaks between launches)."""
    dev = _dev()
    g = torch.Generator().manual_seed(21)
    cases = [((64, 262144), 1024), ((37, 300), 256), ((5, 4097), 1024), ((64, 262144), 1024),
             ((129, 2), 1)]
    for (rows, cols), block in cases:
        x = (4 * torch.randn(rows, cols, generator=g)).bfloat16()
        _say(f"split back to back: [{rows},{cols}] block={block}")
        _check("logsumexp", x, CG.run("logsumexp", x.to(dev), plan="split", block=block))
    x = (4 * torch.randn(48, 20000, generator=g)).bfloat16()
    xd = x.to(dev)
    out = torch.empty(48, dtype=torch.bfloat16, device=dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out.copy_(CG.run("logsumexp", xd, plan="split"))
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out.copy_(CG.run("logsumexp", xd, plan="split"))
    for replay in range(4):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        _say(f"split graph replay {replay}")
        _check("logsumexp", x, out)
        _check("logsumexp", x, CG.run("logsumexp", xd, plan="split"))   # eager in between


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_log_softmax_readout(dtype):
    """run_log_softmax = x - logsumexp(x) per row, fp32, rounded once to x.dtype."""
    dev = _dev()
    g = torch.Generator().manual_seed(21)
    for rows, width in ((5, 1), (33, 77), (16, 1000), (3, 5000), (4, 40000)):
        x = (4 * torch.randn(rows, width, generator=g)).to(dtype)
        _say(f"log_softmax readout {dtype} [{rows},{width}]")
        got = CG.run_log_softmax(x.to(dev)).cpu()
        z = x.float()
        want = z - torch.logsumexp(z, -1, keepdim=True)
        assert got.dtype == dtype and got.shape == x.shape
        if dtype == torch.float32:
            scale = want.abs().amax().item() + 1.0
            torch.testing.assert_close(got, want, rtol=1e-5, atol=2e-6 * scale)
        else:
            # one rounding of a value within a few fp32 ulps of the exact one: <= 1 storage ulp
            ref = want.to(dtype).float()
            ulp = torch.finfo(dtype).eps * want.abs().clamp_min(torch.finfo(dtype).tiny)
            assert ((got.float() - ref).abs() <= ulp * 1.01 + 1e-30).all()
    xs = torch.randn(64, 96, generator=g)[:, ::3].to(dtype)          # strided columns
    _say(f"log_softmax readout strided {dtype}")
    got = CG.run_log_softmax(xs.to(dev)).cpu().float()
    want = torch.log_softmax(xs.float(), -1)
    torch.testing.assert_close(got, want.to(dtype).float(), **dict(zip(("rtol", "atol"), TOL[dtype])))


def test_log_softmax_readout_nonfinite_rows():
    """+inf rows read out NaN (the lowering's where(lse == inf, nan, x - lse)); NaN rows NaN;
    all -inf rows NaN (-inf - -inf); -inf elements of finite rows -inf."""
    dev = _dev()
    x = torch.randn(6, 300, generator=torch.Generator().manual_seed(22))
    x[0, 7] = float("inf")
    x[1, 9] = float("nan")
    x[2] = float("-inf")
    x[3, :150] = float("-inf")
    x[4, 0] = float("inf")
    x[4, 1] = float("-inf")
    got = CG.run_log_softmax(x.to(dev)).cpu()
    lse = torch.logsumexp(x, -1, keepdim=True)
    want = torch.where(lse == float("inf"), float("nan"), x - lse)
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    ok = ~torch.isnan(want)
    torch.testing.assert_close(got[ok], want[ok], rtol=1e-5, atol=1e-5)
    plain = CG.run_log_softmax(x.to(dev), nan_posinf_rows=False).cpu()
    want_plain = x - lse
    assert torch.equal(torch.isnan(plain), torch.isnan(want_plain))
    ok = ~torch.isnan(want_plain)
    torch.testing.assert_close(plain[ok], want_plain[ok], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("width", [300, 40000])
def test_log_softmax_readout_huge_finite_rows(dtype, width):
    """Rows whose max exceeds ~2.3e38 (m * log2(e) overflows fp32) take the exact fallback,
    in the resident kernel (width 300: from the registers it holds) and in the two-read kernel
    (width 40000): the result is the fp64 log-softmax rounded to the dtype."""
    dev = _dev()
    g = torch.Generator().manual_seed(23)
    x = torch.randn(4, width, generator=g)
    x[0, 5] = 3.0e38
    x[1, width - 1] = -3.0e38
    x[1, 2] = 2.5e38
    x[2, :] = 3.0e38
    x = x.to(dtype)
    _say(f"log_softmax readout huge rows {dtype} width {width}")
    got = CG.run_log_softmax(x.to(dev)).cpu()
    z = x.double()
    want = (z - torch.logsumexp(z, -1, keepdim=True)).to(dtype)   # -3e38 - 2.5e38 is -inf
    assert not torch.isnan(got).any()
    torch.testing.assert_close(got.float(), want.float(), **dict(zip(("rtol", "atol"), TOL[dtype])))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_readout_resident_and_two_read_kernels_agree_bit_for_bit(dtype):
    """For one launch shape the resident kernel (row held in registers) and the two-read kernel
    fold the same slots in the same order, so their outputs are identical; rows include -inf,
    +inf (read out NaN) and NaN."""
    from neptune_codegen import hip
    from neptune_codegen import template as T

    dev = _dev()
    g = torch.Generator().manual_seed(24)
    rows, width = 37, 3000
    x = (4 * torch.randn(rows, width, generator=g))
    x[3, 10] = float("inf")
    x[4, 11] = float("nan")
    x[5, :100] = float("-inf")
    x = x.to(dtype).to(dev)
    prog = CG.compile_readout("logsumexp")
    block, warps = CG.best_config(rows, width, x.dtype, x.device)
    var = T._fold_variant(x, width, block, warps, resident=True)
    assert width <= T.readout_tile(var)
    outs = []
    for resident in (True, False):
        out = torch.empty_like(x)
        _say(f"readout kernel resident={resident} {dtype} {var.tag()}")
        prog.kernel(var, 0, resident=resident).launch(
            (T._grid_1d(rows, max(1, var.wg // var.tpr)),),
            (x.data_ptr(), out.data_ptr(), rows, width, x.stride(0), x.stride(1)),
            hip.current_stream(x.device))
        outs.append(out)
    torch.cuda.synchronize()
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(outs[0].view(bits), outs[1].view(bits))
    # run_log_softmax picks the same launch shape and, for this width, the resident kernel
    assert torch.equal(outs[0].view(bits), CG.run_log_softmax(x).view(bits))
    assert torch.isnan(outs[0][3]).all() and torch.isnan(outs[0][4]).all()


def test_log_softmax_graph_through_apply():
    """neptune_opt.apply with the experimental log_softmax lowering runs one readout op on the
    device and verifies against torch (16-bit outputs within 2 ULP)."""
    import neptune_opt

    dev = _dev()

    class LS(torch.nn.Module):
        def forward(self, x):
            return torch.log_softmax(x, dim=-1)

    x = (4 * torch.randn(512, 4096, generator=torch.Generator().manual_seed(23))).bfloat16().to(dev)
    model = LS().eval()
    ep = torch.export.export(model, (x,))
    report = neptune_opt.apply(ep, verify_with=(model, (x,)), experimental_log_softmax=True,
                               max_ulps=2)
    _say(report.summary())
    assert report.fusions and report.verified is True
    targets = [str(n.target) for n in ep.graph_module.graph.nodes if n.op == "call_function"]
    assert targets == ["neptune.logsumexp_tiny0_readout_nanrows.default"], targets
