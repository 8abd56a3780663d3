"""GPU parity at the full sizes the benchmark times, on the benchmark's own seeded inputs.

Every element of each timed workload is checked, not a row sample:
  cfg2 bf16 logsumexp, 16384 x 32000 (the headline's dominant kernel): BASELINE tolerance
      (rtol 1.6e-2 / atol 1e-3) and within one bf16 ulp of the fp32 oracle on every row;
  cfg3 bf16 L2-normalize, 32768 x 4096: BASELINE tolerance against F.normalize in fp32;
  cfg4 fp16 segment sum / mean, 65536 segments, int32 offsets (as drawn, and with empty
      segments injected): bit-exact against torch.segment_reduce on the CPU (the reference
      test's own oracle, tests/test_autotune.py:793-833) and against the C restatement of the
      ordered rounding;
  cfg5 bf16 causal attention, B=4 H=32 S=4096 D=128: all 128 (batch, head) pairs, output
      (bf16 tolerance) and logsumexp (fp32 tolerance), against the fp32 closed form.
Seeds and generators are the ones bench.py uses, so these are the benchmark's inputs.
"""
import math

import numpy as np
import pytest
import torch

import neptune_codegen as CG
from oracle import references as R

pytestmark = pytest.mark.gpu
# The attention fold's row sum adds the fp32 P values: its logsumexp side output is an fp32
# result, held to BASELINE.json's fp32 tolerance.
LSE_RTOL, LSE_ATOL = 1e-5, 1e-6


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda:0")


def _say(*a):
    print(*a, flush=True)


def _seeded(seed):
    return torch.Generator().manual_seed(seed)


def test_cfg2_w32000_all_rows():
    dev = _dev()
    g = _seeded(1)
    for w in (128, 1000, 4096):      # bench.py draws the widths in this order from one stream
        torch.randn(16384, w, generator=g)
    x = (4 * torch.randn(16384, 32000, generator=g)).bfloat16()
    _say("cfg2 logsumexp bf16 [16384,32000], every row")
    got = CG.run("logsumexp", x.to(dev)).cpu().float()
    want = torch.empty(16384)
    for r in range(0, 16384, 2048):            # fp32 oracle in slices (2 GB at once otherwise)
        want[r:r + 2048] = R.reference("logsumexp", x[r:r + 2048])
    torch.testing.assert_close(got, want.bfloat16().float(), rtol=1.6e-2, atol=1e-3)
    # one rounding of the fp32 result: within one bf16 ulp of it on every row
    torch.testing.assert_close(got, want, rtol=torch.finfo(torch.bfloat16).eps, atol=1e-6)


def test_cfg3_l2_normalize_full():
    dev = _dev()
    g = _seeded(3)
    x = torch.randn(32768, 4096, generator=g).bfloat16()
    _say("cfg3 l2-normalize bf16 [32768,4096]")
    got = CG.run_l2_normalize(x.to(dev), eps=1e-6).cpu().float()
    for r in range(0, 32768, 8192):
        want = R.l2_normalize_reference(x[r:r + 8192], 1e-6).float()
        torch.testing.assert_close(got[r:r + 8192], want, rtol=1.6e-2, atol=1e-3)


def _raw16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("empties", [False, True])
@pytest.mark.parametrize("reduce", ["sum", "mean"])
def test_cfg4_all_segments_bit_exact(reduce, empties):
    """The bench's cfg4 input as drawn (Poisson(20) lengths: no empty segment occurs in 65536
    draws), and the same lengths with every 97th segment emptied (empty sums are 0, empty
    means NaN)."""
    from oracle import exact as OX

    dev = _dev()
    g = _seeded(4)
    lengths = torch.poisson(torch.full((65536,), 20.0), generator=g).clamp(0, 200).to(torch.int32)
    total = int(lengths.sum())
    data = torch.randn(total, 128, generator=g).half()
    if empties:
        lengths[::97] = 0
        data = data[:int(lengths.sum())]
    offsets = torch.cat([torch.zeros(1, dtype=torch.int32), lengths.cumsum(0).to(torch.int32)])
    _say(f"cfg4 segment_{reduce} fp16 65536 segments, T={data.shape[0]}, int32 offsets, "
         f"{int((lengths == 0).sum())} empty")
    got = CG.run_segment_pool(data.to(dev), offsets.to(dev), reduce=reduce, offsets=True).cpu()
    want = R.segment_reference(data, offsets, reduce, offsets=True)
    assert got.shape == want.shape == (65536, 128) and got.dtype == torch.float16
    gn, wn = torch.isnan(got), torch.isnan(want)
    assert torch.equal(gn, wn), "NaN (empty-segment) positions differ"
    if empties and reduce == "mean":
        assert bool(gn[::97].all())
    assert torch.equal(got.masked_fill(gn, 0).view(torch.int16), want.masked_fill(wn, 0).view(torch.int16))
    c = OX.segment_pool(_raw16(data), offsets.to(torch.int64).numpy(), "float16", mean=reduce == "mean",
                        initial=None)
    cw = torch.from_numpy(c.view(np.int16)).view(torch.float16)
    cn = torch.isnan(cw)
    assert torch.equal(cn, gn)
    assert torch.equal(got.masked_fill(gn, 0).view(torch.int16), cw.masked_fill(cn, 0).view(torch.int16))
    # lengths form of the same op (the HIP prefix sum builds the spans)
    got_l = CG.run_segment_pool(data.to(dev), lengths.to(dev), reduce=reduce).cpu()
    assert torch.equal(torch.isnan(got_l), gn)
    assert torch.equal(got_l.masked_fill(gn, 0).view(torch.int16), got.masked_fill(gn, 0).view(torch.int16))


def test_cfg5_every_head():
    """cfg5 at full size, every one of the 128 (batch, head) pairs against the fp32 closed
    form: O to the bf16 tolerance, the logsumexp to the fp32 tolerance (8 heads per CPU batch)."""
    dev = _dev()
    g = _seeded(5)
    B, H, S, D = 4, 32, 4096, 128
    q, k, v = (torch.randn(B, H, S, D, generator=g).bfloat16() for _ in range(3))
    _say("cfg5 attention causal [4,32,4096,128], all 128 heads checked")
    out, lse = CG.run_attention(q.to(dev), k.to(dev), v.to(dev), causal=True, return_lse=True)
    out, lse = out.cpu(), lse.cpu()
    mask = torch.ones(S, S, dtype=torch.bool).tril(0)
    for b in range(B):
        for h0 in range(0, H, 8):
            _say(f"  heads b={b} h={h0}..{h0 + 7}")
            qs, ks, vs = (t[b:b + 1, h0:h0 + 8] for t in (q, k, v))
            want = R.attention_reference(qs, ks, vs, causal=True).float()
            torch.testing.assert_close(out[b:b + 1, h0:h0 + 8].float(), want, rtol=1.6e-2, atol=1e-3)
            s = torch.matmul(qs.float(), ks.float().transpose(-1, -2).contiguous()) / math.sqrt(D)
            s = s.masked_fill(~mask, float("-inf"))
            torch.testing.assert_close(lse[b:b + 1, h0:h0 + 8], torch.logsumexp(s, -1),
                                       rtol=LSE_RTOL, atol=LSE_ATOL)
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
