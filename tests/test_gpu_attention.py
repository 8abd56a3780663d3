"""GPU parity of the online-softmax attention fold against the fp32 closed form.

Tolerance: bf16 rtol 1.6e-2 / atol 1e-3, against
softmax(scale * Q K^T + torch is_causal mask) V computed in fp32 on the CPU.
"""
import math

import pytest
import torch

import neptune_codegen as CG
from neptune_codegen import hip
from neptune_codegen.emitters import BASE_OPTIONS, kernel_header
from oracle import references as R

pytestmark = pytest.mark.gpu
# The fold's row sum l adds the fp16-rounded P values that the P.V MFMA multiplies (so O is
# normalised by exactly the weights it used).  A normal fp16 rounding errs by at most 2^-11
# relative (fp16's unit roundoff); a subnormal one (P < 2^-14) by at most 2^-25 absolute.  The
# row's largest P is >= 1, so l >= 1, and for at most 4096 keys the logsumexp m + log(l) is
# within -log(1 - 2^-11) + 4096 * 2^-25 (+ fp32 rounding of m + log l) of the fp32 value.
LSE_ATOL = -math.log1p(-2.0 ** -11) + 4096 * 2.0 ** -25 + 1e-6


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda:0")


def _say(*a):
    print(*a, flush=True)


def test_mfma_32x32x16_bf16_accumulator_layout():
    """The kernel relies on: A lane l holds row l%32 with k = 8*(l/32)+i; B lane l holds column
    l%32 with the same k; accumulator register r of lane l is C[8*(r/4) + 4*(l/32) + r%4][l%32]."""
    dev = _dev()
    src = kernel_header("nep_device.h", "nep_attention.h") + r'''
extern "C" __global__ void mfma_probe(const __bf16* a, const __bf16* b, float* c) {
  const int l = threadIdx.x, m = l & 31, hi = l >> 5;
  nep::bf16x8 av, bv;
  for (int i = 0; i < 8; ++i) {
    av[i] = a[m * 16 + 8 * hi + i];        // A is 32 x 16, row-major
    bv[i] = b[(8 * hi + i) * 32 + m];      // B is 16 x 32, row-major
  }
  nep::f32x16 acc = {};
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
  for (int r = 0; r < 16; ++r) c[(8 * (r / 4) + 4 * hi + (r % 4)) * 32 + m] = acc[r];
}
'''
    prog = hip.Program(src, "mfma_probe.hip", BASE_OPTIONS)
    k = prog.kernel("mfma_probe", (hip.PTR,) * 3, 64, 0)
    g = torch.Generator().manual_seed(11)
    a = torch.randint(-4, 5, (32, 16), generator=g).to(torch.bfloat16)
    b = torch.randint(-4, 5, (16, 32), generator=g).to(torch.bfloat16)
    c = torch.empty(32, 32, device=dev)
    ad, bd = a.to(dev), b.to(dev)
    k.launch((1,), (ad.data_ptr(), bd.data_ptr(), c.data_ptr()), hip.current_stream(dev))
    torch.testing.assert_close(c.cpu(), a.float() @ b.float(), rtol=0, atol=0)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(1, 2, 256, 256, 128), (2, 3, 200, 200, 128), (1, 1, 77, 77, 128),
                                   (1, 2, 130, 333, 64), (1, 1, 1, 64, 128), (1, 4, 512, 512, 64),
                                   (1, 2, 333, 130, 128), (2, 1, 700, 65, 64)])
def test_attention_parity(shape, causal):
    dev = _dev()
    B, H, Sq, Sk, D = shape
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, H, Sq, D, generator=g).bfloat16()
    k = torch.randn(B, H, Sk, D, generator=g).bfloat16()
    v = torch.randn(B, H, Sk, D, generator=g).bfloat16()
    _say(f"attention {shape} causal={causal}")
    got, lse = CG.run_attention(q.to(dev), k.to(dev), v.to(dev), causal=causal, return_lse=True)
    want = R.attention_reference(q, k, v, causal=causal)
    torch.testing.assert_close(got.cpu().float(), want.float(), rtol=1.6e-2, atol=1e-3)
    s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) / math.sqrt(D)
    if causal:
        s = s.masked_fill(~torch.ones(Sq, Sk, dtype=torch.bool).tril(0), float("-inf"))
    torch.testing.assert_close(lse.cpu(), torch.logsumexp(s, -1), rtol=1e-5, atol=LSE_ATOL)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_large_values_use_scaled_tiles(causal):
    """V tiles whose largest |v| reaches 2^15 are packed as v * 2^-e and the fold rescales the
    accumulator around them.  Covers: a tile with max exactly 2^15 (e = 1), one with 1e6 and
    tiny values in other dims, the largest bf16 below 2^16 in the ragged last tile, and a
    tile just below the threshold (e = 0)."""
    dev = _dev()
    g = torch.Generator().manual_seed(12)
    B, H, S, D = 1, 2, 300, 128
    q = torch.randn(B, H, S, D, generator=g).bfloat16()
    k = torch.randn(B, H, S, D, generator=g).bfloat16()
    v = torch.randn(B, H, S, D, generator=g)
    v[0, 0, 5, 3] = 32768.0                      # tile 0: max exactly 2^15
    v[0, 0, 70, 0] = 1.0e6                       # tile 1: large ...
    v[0, 0, 71, 1:9] = 3.0e-4                    # ... next to small values in other dims
    v[0, 0, 299, 7] = -65280.0                   # ragged tile 4: largest bf16 below 2^16
    v[0, 1, 130, 2] = 32512.0                    # tile 2 of head 1: just below 2^15
    v = v.bfloat16()
    _say(f"attention large-|v| tiles causal={causal}")
    got = CG.run_attention(q.to(dev), k.to(dev), v.to(dev), causal=causal)
    want = R.attention_reference(q, k, v, causal=causal)
    torch.testing.assert_close(got.cpu().float(), want.float(), rtol=1.6e-2, atol=1e-3)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_largest_accepted_v_tile_next_to_masked_and_normal_keys(causal):
    """Tiles holding |v| just below 2^28 (tile exponent 13, the largest accepted): packed as
    v * 2^-13, fed P * 2^13 with a row-sum weight of 2^-13, the reference max held 6 higher.
    The tile's other values keep 2^-12 absolute precision -- also on causal rows that see the
    tile but not its large key (queries 64-99 for the key at 100) -- and later tiles' P stay
    within fp16's normal range down to 2^-8 of their unlifted value."""
    dev = _dev()
    g = torch.Generator().manual_seed(13)
    B, H, S, D = 1, 1, 400, 128
    q = torch.randn(B, H, S, D, generator=g).bfloat16()
    k = torch.randn(B, H, S, D, generator=g).bfloat16()
    v = torch.randn(B, H, S, D, generator=g)
    v[0, 0, 100, 3] = 2.0 ** 27 * 1.9921875          # largest bf16 below 2^28
    v[0, 0, 5, 9] = -2.0 ** 27                        # tile 0, another exponent-13 tile
    v = v.bfloat16()
    _say(f"attention exponent-13 V tiles causal={causal}")
    out, lse, status = CG.launch_attention(q.to(dev), k.to(dev), v.to(dev), causal=causal)
    assert status.item() == 1
    want = R.attention_reference(q, k, v, causal=causal).float()
    got = out.cpu().float()
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got, want, rtol=1.6e-2, atol=1e-3)


def test_attention_refuses_v_out_of_range_through_its_status_word():
    """|v| >= 2^28 or inf/NaN in V clear the status word that run_attention asserts on (read
    back here instead, so no device-side assert fires); in-range inputs leave it set."""
    dev = _dev()
    g = torch.Generator().manual_seed(14)
    q, k, v = (torch.randn(1, 2, 200, 64, generator=g).bfloat16() for _ in range(3))
    for value, expected in ((2.0 ** 27, 1), (2.0 ** 28, 0), (2.0 ** 40, 0), (float("inf"), 0),
                            (float("nan"), 0), (-(2.0 ** 100), 0)):
        bad = v.clone()
        bad[0, 1, 150, 7] = value
        _say(f"attention V range status, v={value}")
        _, _, status = CG.launch_attention(q.to(dev), k.to(dev), bad.to(dev), causal=True)
        assert status.item() == expected, value


def test_attention_strided_layout_and_scale():
    """[B, S, H, D] storage viewed as [B, H, S, D] (the common projection layout)."""
    dev = _dev()
    g = torch.Generator().manual_seed(6)
    qs = torch.randn(2, 300, 4, 128, generator=g).bfloat16()
    ks = torch.randn(2, 300, 4, 128, generator=g).bfloat16()
    vs = torch.randn(2, 300, 4, 128, generator=g).bfloat16()
    q, k, v = (t.transpose(1, 2) for t in (qs, ks, vs))
    _say("attention strided [B,S,H,D] view, scale 0.05")
    got = CG.run_attention(qs.to(dev).transpose(1, 2), ks.to(dev).transpose(1, 2),
                           vs.to(dev).transpose(1, 2), scale=0.05, causal=True)
    want = R.attention_reference(q, k, v, scale=0.05, causal=True)
    torch.testing.assert_close(got.cpu().float(), want.float(), rtol=1.6e-2, atol=1e-3)


def test_attention_custom_op():
    dev = _dev()
    op = CG.as_attention_op(causal=True)
    g = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(1, 2, 64, 64, generator=g).bfloat16() for _ in range(3))
    got = op(q.to(dev), k.to(dev), v.to(dev))
    torch.testing.assert_close(got.cpu().float(), R.attention_reference(q, k, v).float(),
                               rtol=1.6e-2, atol=1e-3)
