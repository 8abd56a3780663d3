"""GPU parity of RMSNorm, L2-normalize and segment pooling.

RMS/L2: bf16 rtol 1.6e-2 / atol 1e-3 (fp32: 1e-5 / 1e-6) against the canonical fp32-staged
eager forms.  Segment pooling: bit-exact (NaN positions equal) against torch.segment_reduce on
the CPU, over the reference's own case table (tests/test_autotune.py:793-833).
"""
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


def _bits_equal(a, b):
    assert a.shape == b.shape and a.dtype == b.dtype
    an, bn = torch.isnan(a), torch.isnan(b)
    assert torch.equal(an, bn), "NaN positions differ"
    a, b = a.masked_fill(an, 0), b.masked_fill(bn, 0)
    ia = a.view(torch.int16 if a.element_size() == 2 else torch.int32)
    ib = b.view(torch.int16 if b.element_size() == 2 else torch.int32)
    assert torch.equal(ia, ib), f"{(ia != ib).sum().item()} elements differ bitwise"


@pytest.mark.parametrize("plan", ["serial", "split"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_rms_norm_parity(dtype, plan):
    dev = _dev()
    g = torch.Generator().manual_seed(3)
    for rows, width in ((64, 4096), (7, 1000), (3, 1), (5, 20000)):
        x = torch.randn(rows, width, generator=g).to(dtype)
        gamma = (1 + 0.1 * torch.randn(width, generator=g)).to(dtype)
        _say(f"rms {dtype} {plan} [{rows},{width}]")
        got = CG.run_rms_norm(x.to(dev), gamma.to(dev), eps=1e-6, plan=plan)
        want = R.rms_norm_reference(x, gamma, 1e-6)
        rtol, atol = TOL[dtype]
        torch.testing.assert_close(got.cpu().float(), want.float(), rtol=rtol, atol=atol)
        _say(f"l2 {dtype} {plan} [{rows},{width}]")
        got = CG.run_l2_normalize(x.to(dev), eps=1e-6, plan=plan)
        want = R.l2_normalize_reference(x, 1e-6)
        torch.testing.assert_close(got.cpu().float(), want.float(), rtol=rtol, atol=atol)


def test_repeated_rms_and_l2_calls_reuse_their_launch_and_stay_exact():
    """Repeated serial RMSNorm / L2 calls reuse the first call's kernel and launch shape; calls
    that differ in gamma's alignment or stride, x's alignment, or eps must not share it."""
    from oracle import exact as OX

    dev = _dev()
    g = torch.Generator().manual_seed(24)
    x = torch.randn(40, 520, generator=g).bfloat16()
    gam = (1 + 0.1 * torch.randn(2 * 520 + 8, generator=g)).bfloat16()
    xd, gd = x.to(dev), gam.to(dev)
    xs = [xd[:, :512], xd[:, 8:], xd[:, :512], xd[:, 1:513]]
    gammas = [gd[:512], gd[8:520], gd[1:513], gd[:1024:2]]
    for eps in (1e-6, 1e-2, 1e-6):
        for xv in xs:
            for gv in gammas:
                _say(f"rms repeated x+{xv.storage_offset()} gamma+{gv.storage_offset()}/{gv.stride(0)} eps={eps}")
                got = CG.run_rms_norm(xv, gv, eps=eps).cpu()
                want = _from_raw(OX.rms_norm(_raw(xv.cpu().contiguous()), _raw(gv.cpu().contiguous()),
                                             "bfloat16", eps), torch.bfloat16)
                diff = (got.view(torch.int16).int() - want.view(torch.int16).int()).abs().max().item()
                assert diff <= 2, (eps, xv.storage_offset(), gv.storage_offset(), diff)
            got = CG.run_l2_normalize(xv, eps=eps).cpu()
            want = _from_raw(OX.l2_normalize(_raw(xv.cpu().contiguous()), "bfloat16", eps), torch.bfloat16)
            assert (got.view(torch.int16).int() - want.view(torch.int16).int()).abs().max().item() <= 1
    # the split plan: repeated calls take totals and counts from one allocation
    xw = torch.randn(3, 5000, generator=g)
    gw = 1 + 0.1 * torch.randn(5000, generator=g)
    first = CG.run_rms_norm(xw.to(dev), gw.to(dev), eps=1e-6, plan="split")
    for _ in range(3):
        assert torch.equal(CG.run_rms_norm(xw.to(dev), gw.to(dev), eps=1e-6, plan="split"), first)
    want = _from_raw(OX.rms_norm(_raw(xw), _raw(gw), "float32", 1e-6), torch.float32)
    torch.testing.assert_close(first.cpu(), want, rtol=1e-5, atol=1e-6)


def test_rms_cfg3_shape_and_strided_gamma():
    dev = _dev()
    g = torch.Generator().manual_seed(3)
    x = torch.randn(32768, 4096, generator=g).bfloat16()
    gamma = (1 + 0.1 * torch.randn(4096, generator=g)).bfloat16()
    _say("cfg3 rms [32768,4096] bf16")
    got = CG.run_rms_norm(x.to(dev), gamma.to(dev), eps=1e-6).cpu()
    want = R.rms_norm_reference(x, gamma, 1e-6)
    torch.testing.assert_close(got.float(), want.float(), rtol=1.6e-2, atol=1e-3)
    _say("strided x and gamma")
    xs = torch.randn(16, 2048, generator=g).bfloat16()
    gs = (1 + 0.1 * torch.randn(2048, generator=g)).bfloat16()
    got = CG.run_rms_norm(xs.to(dev)[:, ::2], gs.to(dev)[::2], eps=1e-5).cpu()
    want = R.rms_norm_reference(xs[:, ::2], gs[::2], 1e-5)
    torch.testing.assert_close(got.float(), want.float(), rtol=1.6e-2, atol=1e-3)


def test_segment_reference_case_table():
    """The reference's CUDA segment test (tests/test_autotune.py:793-833), bit-exact."""
    dev = _dev()
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        base = torch.full((1027, 2, 6), 0.1, dtype=dtype)
        base[1, 0, 0] = float("inf")
        base[2, 0, 0] = -float("inf")
        base[3, 1, 2] = float("nan")
        base[4, 1, 4] = -float("inf")
        base_dev = base.to(dev)
        for vi, view in enumerate((lambda b: b[:, :, ::2], lambda b: b.transpose(1, 2))):
            data, data_dev = view(base), view(base_dev)
            lengths = torch.tensor([0, 999, 2, 999, 1025, 999, 0, 999], dtype=torch.int32)[::2]
            offsets = torch.tensor([1, 999, 1, 999, 3, 999, 1026, 999], dtype=torch.int64)[::2]
            ldev = torch.tensor([0, 999, 2, 999, 1025, 999, 0, 999], dtype=torch.int32, device=dev)[::2]
            odev = torch.tensor([1, 999, 1, 999, 3, 999, 1026, 999], dtype=torch.int64, device=dev)[::2]
            for initial in (None, 0.0, -2.125):
                for reduce in ("sum", "mean"):
                    for seg, seg_dev, is_off in ((lengths, ldev, False), (offsets, odev, True)):
                        _say(f"segment {dtype} view{vi} initial={initial} {reduce} offsets={is_off}")
                        want = R.segment_reference(data, seg, reduce, offsets=is_off, initial=initial)
                        got = CG.run_segment_pool(data_dev, seg_dev, reduce=reduce, initial=initial,
                                                  offsets=is_off)
                        _bits_equal(got.cpu(), want)
            torch.testing.assert_close(data_dev.cpu(), data, rtol=0, atol=0, equal_nan=True)
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        data = torch.tensor([[1e-40, -0.0], [1e-40, 0.0]], dtype=dtype)
        lengths = torch.tensor([0, 2])
        for reduce in ("sum", "mean"):
            _say(f"segment signed zero / denormal {dtype} {reduce}")
            got = CG.run_segment_pool(data.to(dev), lengths.to(dev), reduce=reduce, initial=-0.0).cpu()
            want = R.segment_reference(data, lengths, reduce, initial=-0.0)
            _bits_equal(got, want)
            assert torch.equal(torch.signbit(got), torch.signbit(want))
    data = torch.zeros(1027, 3, dtype=torch.bfloat16)
    lengths = torch.tensor([1027])
    op = CG.as_segment_op("segment_mean", {"initial": 7.0}, lib="segment_gpu_tests")
    _bits_equal(op(data.to(dev), lengths.to(dev)).cpu(),
                R.segment_reference(data, lengths, "mean", initial=7.0))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_segment_cfg4_vector_path_bit_exact(dtype):
    dev = _dev()
    g = torch.Generator().manual_seed(4)
    lengths = torch.poisson(torch.full((4096,), 20.0), generator=g).clamp(0, 200).to(torch.int32)
    total = int(lengths.sum())
    data = torch.randn(total, 128, generator=g).to(dtype)
    offsets = torch.cat([torch.zeros(1, dtype=torch.int32), lengths.cumsum(0).to(torch.int32)])
    for reduce in ("sum", "mean"):
        _say(f"cfg4-style segment {dtype} {reduce} T={total}")
        got = CG.run_segment_pool(data.to(dev), offsets.to(dev), reduce=reduce, offsets=True).cpu()
        want = R.segment_reference(data, offsets, reduce, offsets=True)
        _bits_equal(got, want)


def _raw(t):
    import numpy as np

    if t.dtype == torch.float32:
        return t.contiguous().numpy()
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _from_raw(a, dtype):
    import numpy as np

    if dtype == torch.float32:
        return torch.from_numpy(a)
    return torch.from_numpy(a.view(np.int16)).view(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_segment_against_c_oracle_and_device_segment_reduce(dtype):
    """Bit-exact against the C restatement of the ordered rounding and against torch's own
    segment_reduce on the device (the CPU-vs-device agreement the reference assumes)."""
    from oracle import exact as OX

    dev = _dev()
    g = torch.Generator().manual_seed(9)
    lengths = torch.poisson(torch.full((512,), 20.0), generator=g).clamp(0, 200).to(torch.int64)
    lengths[::37] = 0
    data = (2 * torch.randn(int(lengths.sum()), 128, generator=g)).to(dtype)
    data[5, 3] = float("inf")
    data[17, 9] = float("nan")
    spans = torch.cat([torch.zeros(1, dtype=torch.int64), lengths.cumsum(0)])
    for reduce, initial in (("sum", None), ("mean", None), ("sum", -2.125), ("mean", 7.0)):
        _say(f"segment vs C oracle {dtype} {reduce} initial={initial}")
        got = CG.run_segment_pool(data.to(dev), spans.to(dev), reduce=reduce, offsets=True,
                                  initial=initial).cpu()
        want = _from_raw(OX.segment_pool(_raw(data), spans.numpy(), str(dtype).split(".")[1],
                                         mean=reduce == "mean", initial=initial), dtype)
        _bits_equal(got, want)
        on_dev = torch.segment_reduce(data.to(dev), reduce, axis=0, offsets=spans.to(dev),
                                      initial=initial).cpu()
        _bits_equal(got, on_dev)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rms_l2_against_c_oracle(dtype):
    """Against the C restatement of the staged arithmetic (fp32 sum of squares, correctly
    rounded division and rsqrt, rounding before gamma): equal up to the summation order, so
    almost every element matches bit for bit; RMS rounds twice (normalized, then times gamma),
    so a one-ulp difference in the statistics can reach two ulps of the output."""
    import numpy as np

    from oracle import exact as OX

    dev = _dev()
    g = torch.Generator().manual_seed(3)
    x = torch.randn(256, 4096, generator=g).to(dtype)
    gamma = (1 + 0.1 * torch.randn(4096, generator=g)).to(dtype)
    name = str(dtype).split(".")[1]
    for which in ("rms", "l2"):
        _say(f"{which} vs C oracle {dtype}")
        if which == "rms":
            got = CG.run_rms_norm(x.to(dev), gamma.to(dev), eps=1e-6).cpu()
            want = _from_raw(OX.rms_norm(_raw(x), _raw(gamma), name, 1e-6), dtype)
        else:
            got = CG.run_l2_normalize(x.to(dev), eps=1e-6).cpu()
            want = _from_raw(OX.l2_normalize(_raw(x), name, 1e-6), dtype)
        same = (got.view(torch.int16) == want.view(torch.int16)).float().mean().item()
        assert same > 0.98, same
        ulps = (got.view(torch.int16).int() - want.view(torch.int16).int()).abs().max().item()
        assert ulps <= 2, ulps


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_l2_division_by_the_row_norm_is_correctly_rounded(dtype):
    """The L2 readout divides by the row norm through its reciprocal and one exact FMA
    correction, and hands elements outside that method's exact range to the correctly rounded
    division: nonzero |v| < 2^-100, quotients below 2^-125 of the norm, rows whose sum of
    squares overflows.  Rows whose sum of squares is exact in any order (small integers, powers
    of two) fix the norm, so the output must equal the C oracle's correctly rounded division
    bit for bit, signed zeros included."""
    import numpy as np

    from oracle import exact as OX

    dev = _dev()
    g = torch.Generator().manual_seed(31)
    w = 4096
    x = torch.zeros(6, w)
    x[0] = torch.randint(-7, 8, (w,), generator=g).float()            # integers: exact squares
    x[0, 10:16] = torch.tensor([2.0 ** -110, -2.0 ** -120, 2.0 ** -126, 0.0, -0.0, 2.0 ** -100])
    x[1] = torch.randint(-7, 8, (w,), generator=g).float()
    x[1, 100] = 2.0 ** 100                                             # squares overflow: norm inf
    x[1, 101] = -3.0
    x[2, :4] = 2.0 ** 60                                               # norm 2^61
    x[2, 4:12] = torch.tensor([2.0 ** -80, -2.0 ** -90, 3.0, -5.0, 7.0, 2.0 ** 40, -0.0, 1.0])
    x[3, 7] = -0.0                                                     # norm 0: divided by eps
    x[4] = torch.randint(-3, 4, (w,), generator=g).float() * 2.0 ** -60
    x[5] = torch.randn(w, generator=g)
    x = x.to(dtype)
    name = str(dtype).split(".")[1]
    _say(f"l2 division edge rows {dtype}")
    got = CG.run_l2_normalize(x.to(dev), eps=1e-6).cpu()
    want = _from_raw(OX.l2_normalize(_raw(x), name, 1e-6), dtype)
    view = torch.int16 if dtype != torch.float32 else torch.int32
    gb, wb = got.view(view), want.view(view)
    assert torch.equal(gb[:5], wb[:5]), (gb[:5] != wb[:5]).nonzero()[:8].tolist()
    assert torch.isfinite(got).all()
    assert (got[1] == 0).all() and bool(torch.signbit(got[1, 101]))   # v / inf = -0 for v < 0
    assert bool(torch.signbit(got[0, 14])) and bool(torch.signbit(got[3, 7]))
    # the random row: equal up to the summation order of its norm (one output ulp in bf16;
    # fp32 keeps that order difference, within the fp32 tolerance)
    if dtype == torch.float32:
        torch.testing.assert_close(got[5], want[5], rtol=1e-5, atol=1e-6)
    else:
        assert (gb[5].int() - wb[5].int()).abs().max().item() <= 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_l2_norm_whose_reciprocal_is_not_normal_takes_the_exact_division(dtype):
    """eps is any finite positive number: a denormal eps under a row whose squares all
    underflow (norm = eps = 1e-40, reciprocal overflows), and eps >= 2^126 (reciprocal
    denormal).  The fast reciprocal path does not hold there; the rows must still equal the
    C oracle's correctly rounded division bit for bit."""
    from oracle import exact as OX

    dev = _dev()
    name = str(dtype).split(".")[1]
    view = torch.int16 if dtype != torch.float32 else torch.int32
    w = 512
    tiny_row = torch.zeros(2, w)
    tiny_row[0, ::3] = 2.0 ** -90                   # squares 2^-180 underflow to 0
    tiny_row[0, 1::7] = -(2.0 ** -80)
    tiny_row[1, 5] = 2.0 ** -75
    big_eps_rows = torch.randint(-40, 41, (2, w), generator=torch.Generator().manual_seed(33)).float()
    for x, eps in ((tiny_row, 1e-40), (big_eps_rows, 1e38), (big_eps_rows * 2.0 ** 50, 2.0 ** 127)):
        x = x.to(dtype)
        _say(f"l2 eps={eps} {dtype}")
        got = CG.run_l2_normalize(x.to(dev), eps=eps).cpu()
        want = _from_raw(OX.l2_normalize(_raw(x), name, eps), dtype)
        assert torch.isfinite(got).all()
        assert torch.equal(got.view(view), want.view(view)), (got.view(view) != want.view(view)).nonzero()[:8].tolist()


def test_repeated_segment_calls_reuse_their_launch_and_stay_exact():
    """Repeated CSR-offset segment calls with the same layout reuse the first call's kernel and
    launch shape; other offset values, another data alignment or another reduction must give
    the C oracle's ordered results bit for bit."""
    from oracle import exact as OX

    dev = _dev()
    g = torch.Generator().manual_seed(25)
    data = torch.randn(1001, 64, generator=g).bfloat16()
    dd = data.to(dev)
    for trial in range(3):
        lengths = torch.randint(0, 40, (30,), generator=g)
        offsets = torch.cat([torch.zeros(1, dtype=torch.int64), lengths.cumsum(0)])
        offsets = offsets.clamp(max=1000)
        for view, cpu in ((dd[:1000], data[:1000]), (dd[1:], data[1:])):
            for reduce in ("sum", "mean", "sum"):
                _say(f"segment repeated trial {trial} {reduce} offset {view.storage_offset()}")
                got = CG.run_segment_pool(view, offsets.to(dev), reduce=reduce, offsets=True).cpu()
                ref = _from_raw(OX.segment_pool(_raw(cpu.contiguous()), offsets.numpy(), "bfloat16",
                                                mean=reduce == "mean", initial=None), torch.bfloat16)
                assert torch.equal(torch.nan_to_num(got, 7.0), torch.nan_to_num(ref, 7.0)), (trial, reduce)
    # int32 offsets and rank-3 data (channels flattened): other keys, same contract
    data3 = torch.randn(600, 4, 16, generator=g).half()
    for trial in range(2):
        lengths = torch.randint(0, 30, (25,), generator=g)
        off32 = torch.cat([torch.zeros(1, dtype=torch.int32), lengths.cumsum(0).to(torch.int32)]).clamp(max=600)
        got = CG.run_segment_pool(data3.to(dev), off32.to(dev), reduce="sum", offsets=True).cpu()
        ref = _from_raw(OX.segment_pool(_raw(data3.reshape(600, 64)), off32.numpy().astype("int64"),
                                        "float16", mean=False, initial=None), torch.float16)
        assert got.shape == (25, 4, 16)
        assert torch.equal(got.reshape(25, 64), ref), trial


def test_segment_fused_descriptor_check_matches_reference_asserts():
    """The span checks fused into the segment kernel clear the status word exactly when the
    reference's asserts (range, coverage unless unsafe, monotonic; torch_op.py:378-386, run here
    on the CPU by _segment_spans) would fail.  Malformed spans issue no loads, so the launches
    are safe; the status is read back instead of being asserted on the device."""
    from neptune_codegen import torch_op as TO

    dev = _dev()
    data = torch.randn(7, 16).half()
    program = CG.compile_segment_reduction("segment_sum", {"offsets": False})
    program_off = CG.compile_segment_reduction("segment_sum", {"offsets": True})
    cases = [([0, 2, 0, 5], False, False), ([7], False, False), ([3, 4], False, False),
             ([-1, 8], False, False), ([3, 3], False, False), ([8], False, True), ([4, 4], False, True),
             ([2, 2], False, True), ([5, -1, 3], False, False), ([0, 3, 7], True, False),
             ([0, 3, 3, 7], True, True), ([-1, 4], True, True), ([0, 8], True, False),
             ([4, 3], True, True), ([2, 5], True, False), ([0, 7, 6], True, False)]
    for indices, is_offsets, unsafe in cases:
        for idx_dtype in (torch.int32, torch.int64):
            seg = torch.tensor(indices, dtype=idx_dtype)
            try:
                TO._segment_spans(data, seg, offsets=is_offsets, unsafe=unsafe)
                reference_ok = True
            except RuntimeError:
                reference_ok = False
            _say(f"fused descriptor check {indices} offsets={is_offsets} unsafe={unsafe} {idx_dtype}")
            seg_dev = seg.to(dev)
            status = torch.zeros(1, dtype=torch.int32, device=dev)
            spans, status_set = TO._device_spans(data, seg_dev, offsets=is_offsets, status=status)
            assert status_set == (not is_offsets)
            if not status_set:
                status.fill_(1)
            nseg = spans.shape[0] - 1
            out = torch.empty(nseg, 16, dtype=torch.float16, device=dev)
            cover = -1 if is_offsets or unsafe else data.shape[0]
            TO.launch_segment_kernel(program_off if is_offsets else program, data.to(dev), spans, out,
                                     status=status, cover=cover)
            assert bool(status.item()) == reference_ok, (indices, is_offsets, unsafe)
            if reference_ok:
                want = R.segment_reference(data, seg, "sum", offsets=is_offsets, unsafe=unsafe)
                _bits_equal(out.cpu(), want)


@pytest.mark.parametrize("dtype", [torch.int32, torch.int64])
def test_lengths_prefix_sum_kernel_is_exact(dtype):
    """The HIP lengths -> spans scan equals cat(0, cumsum(lengths)) exactly, across block
    boundaries (1024 lengths per workgroup) and with zero and very large lengths."""
    from neptune_codegen.torch_op import _device_spans

    dev = _dev()
    g = torch.Generator().manual_seed(41)
    for n in (1, 5, 1023, 1024, 1025, 65536, 1_000_003):
        lengths = torch.randint(0, 201, (n,), generator=g).to(dtype)
        lengths[::7] = 0
        if dtype == torch.int64:
            lengths[n // 2] = 1 << 40
        print(f"spans scan {dtype} n={n}", flush=True)
        status = torch.zeros(1, dtype=torch.int32, device=dev)
        got, status_set = _device_spans(None, lengths.to(dev), offsets=False, status=status)
        want = torch.cat([torch.zeros(1, dtype=torch.int64), lengths.to(torch.int64).cumsum(0)])
        assert got.dtype == torch.int64 and torch.equal(got.cpu(), want)
        assert status_set and status.item() == 1, "the first spans launch sets the status word"


def test_segment_status_word_is_armed_once_and_graph_capture_before_it_exists():
    """The segment op's span-check status word is armed once per device, outside capture.  A
    first call under graph capture (no word yet) arms a word of its own in the captured
    stream; replays and later eager calls give the reference results and leave the device
    word set."""
    from neptune_codegen import torch_op as TO

    dev = _dev()
    g = torch.Generator().manual_seed(21)
    data = torch.randn(300, 128, generator=g).half()
    lengths = torch.tensor([0, 5, 120, 0, 75, 100], dtype=torch.int32)
    want = R.segment_reference(data, lengths, "sum")
    d_dev, l_dev = data.to(dev), lengths.to(dev)
    TO._STATUS.pop(0, None)
    _say("segment op: first call under graph capture")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            out = CG.run_segment_pool(d_dev, l_dev, reduce="sum")
    torch.cuda.current_stream().wait_stream(s)
    assert 0 not in TO._STATUS
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        _bits_equal(out.cpu(), want)
    _say("segment op: eager calls arm the device word")
    for reduce in ("sum", "mean", "sum"):
        got = CG.run_segment_pool(d_dev, l_dev, reduce=reduce)
        _bits_equal(got.cpu(), R.segment_reference(data, lengths, reduce))
    assert TO._STATUS[0].item() == 1
