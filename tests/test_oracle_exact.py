"""Pins of the C oracle (oracle/csrc/neptune_oracle.c) -- CPU only.

  * f32 -> bf16 / fp16 rounding against torch's own conversions over a sweep of fp32 bit
    patterns (all exponents, mantissa ties, subnormals, overflow, NaN/inf);
  * rsqrt_rn against an independent exact-integer midpoint test, exhaustively over [1, 4)
    (rsqrt(4^k x) = 2^-k rsqrt(x) exactly, so [1, 4) covers every positive input whose result
    is normal -- all of them), plus a strided sweep of the whole positive range and the IEEE
    special values;
  * segment pooling bit-exact against the reference's case table (fixtures from
    torch.segment_reduce) and against torch.segment_reduce on random ragged inputs;
  * RMSNorm / L2-normalize against the canonical eager forms.
"""
import json
import math
import pathlib
import struct

import numpy as np
import pytest
import torch

from oracle import exact as OX
from oracle import references as R

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def _sweep_bits(n=400_000, seed=0):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    extra = []
    for e in range(0, 256):
        for m in (0, 1, 0x7fff, 0x8000, 0x8001, 0xffff, 0x1000, 0x0fff, 0x1fff, 0x2000, 0x7fffff, 0x400000):
            for s in (0, 1 << 31):
                extra.append(s | (e << 23) | m)
    return np.concatenate([bits, np.array(extra, np.uint32)])


def test_bf16_rounding_matches_torch():
    bits = _sweep_bits()
    f = bits.view(np.float32)
    got = np.array([OX.lib().nor_f32_to_bf16(float(v)) for v in f[:60000]], np.uint16)
    want = torch.from_numpy(f[:60000].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(f[:60000])
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7fff) > 0x7f80)


def test_f16_rounding_matches_torch():
    bits = _sweep_bits(seed=1)
    f = bits.view(np.float32)[:60000]
    got = np.array([OX.lib().nor_f32_to_f16(float(v)) for v in f], np.uint16)
    want = torch.from_numpy(f.copy()).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], want[~nan]), np.flatnonzero(got[~nan] != want[~nan])[:5]
    # fp16 -> fp32 is exact
    h = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    back = np.array([OX.lib().nor_f16_to_f32(int(v)) for v in h], np.float32)
    tb = torch.from_numpy(h.view(np.int16).copy()).view(torch.float16).float().numpy()
    ok = ~np.isnan(tb)
    assert np.array_equal(back[ok].view(np.uint32), tb[ok].view(np.uint32))


def test_rsqrt_rn_exhaustive_on_one_to_four():
    lo = struct.unpack("I", struct.pack("f", 1.0))[0]
    hi = struct.unpack("I", struct.pack("f", 4.0))[0]
    bad, first = OX.check_rsqrt_range(lo, hi, 1)
    assert bad == 0, f"first incorrectly rounded input bits 0x{first:08x}"


def test_rsqrt_rn_strided_full_range_and_specials():
    bad, first = OX.check_rsqrt_range(1, 0x7f800000, 997)
    assert bad == 0, f"0x{first:08x}"
    f = OX.rsqrt_rn
    assert f(0.0) == math.inf and f(-0.0) == -math.inf
    assert math.isnan(f(-1.0)) and math.isnan(f(float("nan")))
    assert f(float("inf")) == 0.0
    assert f(1.0) == 1.0 and f(4.0) == 0.5 and f(0.25) == 2.0
    # a plausible wrong implementation (fp32 1/sqrtf) is caught by the exact test
    x = np.float32(5.0)
    naive = np.float32(1.0) / np.sqrt(x)
    assert OX.lib().nor_rsqrt_is_correctly_rounded(float(x), float(OX.rsqrt_rn(float(x))))
    wrong = 0
    for v in np.random.default_rng(3).uniform(1, 4, 20000).astype(np.float32):
        nv = np.float32(np.float32(1.0) / np.sqrt(v))
        wrong += not OX.lib().nor_rsqrt_is_correctly_rounded(float(v), float(nv))
    assert wrong > 0, "the exact test must be able to reject a non-correctly-rounded rsqrt"


def _torch_dtype(name):
    return getattr(torch, name)


def test_segment_reference_case_table_bit_exact():
    table = json.loads((GOLDEN / "segment_cases.json").read_text())
    for case in table["cases"]:
        dt = _torch_dtype(case["dtype"])
        if case.get("data") == "signed_zero_denormal":
            data = torch.tensor([[1e-40, -0.0], [1e-40, 0.0]], dtype=dt)
        else:
            base = torch.full((1027, 2, 6), 0.1, dtype=dt)
            base[1, 0, 0] = float("inf")
            base[2, 0, 0] = -float("inf")
            base[3, 1, 2] = float("nan")
            base[4, 1, 4] = -float("inf")
            data = base[:, :, ::2].contiguous().reshape(1027, 6)
        seg = np.array(case["segments"], np.int64)
        spans = seg if case["offsets"] else np.concatenate([[0], np.cumsum(seg)])
        view = torch.int16 if dt != torch.float32 else torch.int32
        raw = data.view(view).numpy()
        raw = raw.view(np.uint16) if dt != torch.float32 else raw.view(np.float32)
        out = OX.segment_pool(raw, spans, case["dtype"], mean=case["reduce"] == "mean",
                              initial=case["initial"])
        ot = torch.from_numpy(out.view(np.int16) if dt != torch.float32 else out).view(dt) \
            if dt != torch.float32 else torch.from_numpy(out)
        nan = torch.isnan(ot.float()).flatten()
        assert nan.tolist() == case["nan"], case
        bits = ot.masked_fill(torch.isnan(ot), 0).view(view).flatten().tolist()
        assert bits == case["bits"], case


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
def test_segment_random_against_torch(dtype):
    dt = _torch_dtype(dtype)
    g = torch.Generator().manual_seed(4)
    lengths = torch.poisson(torch.full((300,), 6.0), generator=g).clamp(0, 40).to(torch.int64)
    data = (3 * torch.randn(int(lengths.sum()), 16, generator=g)).to(dt)
    spans = np.concatenate([[0], np.cumsum(lengths.numpy())])
    view = torch.int16 if dt != torch.float32 else torch.int32
    raw = data.view(view).numpy()
    raw = raw.view(np.uint16) if dt != torch.float32 else raw.view(np.float32)
    for reduce, initial in (("sum", None), ("mean", None), ("sum", 1.5), ("mean", -0.0)):
        out = OX.segment_pool(raw, spans, dtype, mean=reduce == "mean", initial=initial)
        got = torch.from_numpy(out.view(np.int16)).view(dt) if dt != torch.float32 else torch.from_numpy(out)
        want = torch.segment_reduce(data, reduce, axis=0, lengths=lengths, initial=initial)
        assert torch.equal(torch.isnan(got), torch.isnan(want))
        assert torch.equal(got.masked_fill(torch.isnan(got), 0).view(view),
                           want.masked_fill(torch.isnan(want), 0).view(view))


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_rms_and_l2_against_canonical_forms(dtype):
    dt = _torch_dtype(dtype)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(16, 1000, generator=g).to(dt)
    gamma = (1 + 0.1 * torch.randn(1000, generator=g)).to(dt)
    view = torch.int16 if dt != torch.float32 else torch.int32

    def raw(t):
        a = t.contiguous().view(view).numpy()
        return a.view(np.uint16) if dt != torch.float32 else a.view(np.float32)

    def back(a):
        return torch.from_numpy(a.view(np.int16)).view(dt) if dt != torch.float32 else torch.from_numpy(a)

    tol = dict(rtol=1e-5, atol=1e-6) if dt == torch.float32 else dict(rtol=1.6e-2, atol=1e-3)
    rms = back(OX.rms_norm(raw(x), raw(gamma), dtype, 1e-6))
    want = R.rms_norm_reference(x, gamma, 1e-6)
    torch.testing.assert_close(rms.float(), want.float(), **tol)
    if dt != torch.float32:
        # stage order (round to dtype before gamma): in 16-bit storage the final rounding hides
        # summation-order differences, so nearly every element matches torch bit for bit; a
        # gamma applied before the rounding would not
        assert (rms.float() == want.float()).float().mean() > 0.95
        swapped = (x.float() * torch.rsqrt((x.float() ** 2).mean(-1, keepdim=True) + 1e-6) * gamma.float()).to(dt)
        assert (swapped.float() == want.float()).float().mean() < (rms.float() == want.float()).float().mean()
    l2 = back(OX.l2_normalize(raw(x), dtype, 1e-6))
    torch.testing.assert_close(l2.float(), R.l2_normalize_reference(x, 1e-6).float(), **tol)
