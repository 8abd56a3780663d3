"""GPU parity of the online-softmax attention fold against the fp32 closed form.

Tolerance: bf16/fp16 rtol 1.6e-2 / atol 1e-3 for O, against
softmax(scale * Q K^T + torch is_causal mask) V computed in fp32 on the CPU; fp32 rtol 1e-5 /
atol 1e-6 for the logsumexp side output against torch.logsumexp of the same fp32 scores.
"""
import math

import pytest
import torch

import neptune_codegen as CG
from neptune_codegen import attention as A
from neptune_codegen import hip
from neptune_codegen.emitters import BASE_OPTIONS, kernel_header
from oracle import references as R

pytestmark = pytest.mark.gpu
# The row sum l adds the fp32 P values, so the logsumexp side output is an fp32 result:
# BASELINE.json's fp32 tolerance applies.
LSE_RTOL, LSE_ATOL = 1e-5, 1e-6


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


def _lse_reference(q, k, causal, scale=None):
    Sq, Sk, D = q.shape[2], k.shape[2], q.shape[3]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) * scale
    if causal:
        s = s.masked_fill(~torch.ones(Sq, Sk, dtype=torch.bool).tril(0), float("-inf"))
    return torch.logsumexp(s, -1)


SHAPES = [(1, 2, 256, 256, 128), (2, 3, 200, 200, 128), (1, 1, 77, 77, 128),
          (1, 2, 130, 333, 64), (1, 1, 1, 64, 128), (1, 4, 512, 512, 64),
          (1, 2, 333, 130, 128), (2, 1, 700, 65, 64), (1, 2, 300, 300, 256),
          (1, 1, 130, 333, 256), (2, 1, 1, 70, 256)]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", SHAPES)
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
    torch.testing.assert_close(lse.cpu(), _lse_reference(q, k, causal), rtol=LSE_RTOL, atol=LSE_ATOL)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(1, 2, 256, 256, 128), (2, 3, 200, 200, 128), (1, 2, 130, 333, 64),
                                   (1, 1, 1, 64, 128), (2, 1, 700, 65, 64), (1, 2, 200, 200, 256)])
def test_attention_parity_fp16(shape, causal):
    """fp16 Q/K/V: the f16 MFMA for Q K^T, the same fp16 P.V, an fp16 output."""
    dev = _dev()
    B, H, Sq, Sk, D = shape
    g = torch.Generator().manual_seed(15)
    q = torch.randn(B, H, Sq, D, generator=g).half()
    k = torch.randn(B, H, Sk, D, generator=g).half()
    v = (3 * torch.randn(B, H, Sk, D, generator=g)).half()
    _say(f"attention fp16 {shape} causal={causal}")
    got, lse = CG.run_attention(q.to(dev), k.to(dev), v.to(dev), causal=causal, return_lse=True)
    assert got.dtype == torch.float16
    want = R.attention_reference(q, k, v, causal=causal)
    torch.testing.assert_close(got.cpu().float(), want.float(), rtol=1.6e-2, atol=1e-3)
    torch.testing.assert_close(lse.cpu(), _lse_reference(q, k, causal), rtol=LSE_RTOL, atol=LSE_ATOL)


def test_attention_fp16_values_at_the_top_of_the_range():
    """fp16 V holding 65504 and -32768 (tile exponent 1) next to fp16 subnormals."""
    dev = _dev()
    g = torch.Generator().manual_seed(16)
    B, H, S, D = 1, 2, 200, 128
    q, k = (torch.randn(B, H, S, D, generator=g).half() for _ in range(2))
    v = torch.randn(B, H, S, D, generator=g)
    v[0, 0, 10, 5] = 65504.0
    v[0, 1, 150, 0] = -32768.0
    v[0, 1, 151, 1:9] = 2.0 ** -20
    v = v.half()
    _say("attention fp16 top-of-range V")
    out, _, exps = CG.launch_attention(q.to(dev), k.to(dev), v.to(dev), causal=True)
    assert not CG.exact_path_taken(exps)
    torch.testing.assert_close(out.cpu().float(), R.attention_reference(q, k, v, causal=True).float(),
                               rtol=1.6e-2, atol=1e-3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [(1, 2, 256, 256, 128), (1, 1, 300, 333, 64), (2, 1, 77, 77, 128),
                                   (1, 1, 200, 150, 256)])
def test_attention_exact_path_matches_the_fp32_closed_form(shape, causal, dtype):
    """The exact fp32 path (forced for every query block by an exponent threshold of -1): fp32
    scores, fp32 P, the caller's V.  Its O is within the storage rounding of the fp32 closed
    form, and its logsumexp within the fp32 tolerance."""
    dev = _dev()
    B, H, Sq, Sk, D = shape
    g = torch.Generator().manual_seed(17)
    q, k, v = (torch.randn(B, H, n, D, generator=g).to(dtype) for n in (Sq, Sk, Sk))
    _say(f"attention exact path {shape} causal={causal} {dtype}")
    out, lse, _ = A._launch(q.to(dev), k.to(dev), v.to(dev), None, causal, True, -1)
    want = R.attention_reference(q.float(), k.float(), v.float(), causal=causal)
    # one rounding of an fp32 value: half an ulp, 2^-8 (bf16) or 2^-11 (fp16) relative at most
    half_ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    torch.testing.assert_close(out.cpu().float(), want, rtol=1.01 * half_ulp, atol=1e-5)
    torch.testing.assert_close(lse.cpu(), _lse_reference(q, k, causal), rtol=LSE_RTOL, atol=LSE_ATOL)


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
    """Tiles holding |v| just below 2^28 (tile exponent 13, the largest the MFMA path takes):
    packed as v * 2^-13, fed P * 2^13 with a row-sum weight of 2^-13, the reference max held 6
    higher.  The tile's other values keep 2^-12 absolute precision -- also on causal rows that
    see the tile but not its large key (queries 64-99 for the key at 100) -- and later tiles'
    P stay within fp16's normal range down to 2^-8 of their unlifted value."""
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
    out, lse, exps = CG.launch_attention(q.to(dev), k.to(dev), v.to(dev), causal=causal,
                                         return_lse=True)
    assert not CG.exact_path_taken(exps)
    assert exps.cpu().tolist()[:2] == [13, 13]
    want = R.attention_reference(q, k, v, causal=causal).float()
    got = out.cpu().float()
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got, want, rtol=1.6e-2, atol=1e-3)
    torch.testing.assert_close(lse.cpu(), _lse_reference(q, k, causal), rtol=LSE_RTOL, atol=LSE_ATOL)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("value", [2.0 ** 28, -(2.0 ** 40), 2.0 ** 100, 3.0e38])
def test_attention_large_finite_v_takes_the_exact_path(value, causal):
    """|v| >= 2^28 is beyond the fp16 images' range: the pack records the tile's own exponent
    and the query blocks that see the tile take the exact fp32 path.  Rows before the tile
    (causal) stay on the MFMA path; every row matches the fp32 closed form."""
    dev = _dev()
    g = torch.Generator().manual_seed(14)
    B, H, S, D = 1, 2, 600, 64
    q, k = (torch.randn(B, H, S, D, generator=g).bfloat16() for _ in range(2))
    v = torch.randn(B, H, S, D, generator=g)
    v[0, 1, 450, 7] = value
    v[0, 1, 452, 2] = 1e-3
    v = v.bfloat16()
    _say(f"attention large V {value} causal={causal}")
    out, lse, exps = CG.launch_attention(q.to(dev), k.to(dev), v.to(dev), causal=causal,
                                         return_lse=True)
    e = exps.view(B * H, -1).cpu()
    assert int(e[1, 450 // 64]) == int(math.floor(math.log2(abs(float(torch.tensor(value).bfloat16()))))) - 14
    assert CG.exact_path_taken(exps)
    want = R.attention_reference(q, k, v, causal=causal).float()
    got = out.cpu().float()
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got, want, rtol=1.6e-2, atol=1e-3)
    torch.testing.assert_close(lse.cpu(), _lse_reference(q, k, causal), rtol=LSE_RTOL, atol=LSE_ATOL)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("value", [float("inf"), float("-inf"), float("nan")])
def test_attention_non_finite_v_reaches_only_the_rows_that_see_it(value, causal):
    """inf/NaN in V: no error and no trap.  The query blocks that see the tile take the exact
    fp32 path, where masked keys contribute nothing: the rows that see the key get inf/NaN in
    its column (p > 0 times the value), every other value matches the fp32 closed form of the
    keys the row sees."""
    dev = _dev()
    g = torch.Generator().manual_seed(18)
    B, H, S, D = 1, 2, 700, 128
    j, col = 530, 9
    q, k = (torch.randn(B, H, S, D, generator=g).bfloat16() for _ in range(2))
    v = torch.randn(B, H, S, D, generator=g).bfloat16()
    v[0, 0, j, col] = value
    _say(f"attention non-finite V {value} causal={causal}")
    out, lse, exps = CG.launch_attention(q.to(dev), k.to(dev), v.to(dev), causal=causal,
                                         return_lse=True)
    assert CG.exact_path_taken(exps)
    got = out.cpu().float()
    clean = v.clone()
    clean[0, 0, j, col] = 0.0
    want = R.attention_reference(q, k, clean, causal=causal).float()
    sees = torch.zeros(S, dtype=torch.bool)
    sees[j if causal else 0:] = True
    bad = got[0, 0, :, col]
    if math.isnan(value):
        assert torch.isnan(bad[sees]).all()
    else:
        assert (bad[sees] == value).all()
    keep = torch.ones_like(got, dtype=torch.bool)
    keep[0, 0, sees, col] = False
    torch.testing.assert_close(got[keep], want[keep], rtol=1.6e-2, atol=1e-3)
    torch.testing.assert_close(lse.cpu(), _lse_reference(q, k, causal), rtol=LSE_RTOL, atol=LSE_ATOL)


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_rows_whose_scores_are_all_minus_inf(causal, exact):
    """A query holding -inf against keys that are all positive in that dimension scores -inf on
    every key: softmax gives NaN for the row and logsumexp -inf, on the MFMA path and on the
    exact path alike; the other rows are unaffected."""
    dev = _dev()
    g = torch.Generator().manual_seed(20)
    B, H, S, D = 1, 2, 200, 128
    q, k, v = (torch.randn(B, H, S, D, generator=g) for _ in range(3))
    k[..., 3] = k[..., 3].abs() + 0.5
    q[0, 1, 150, 3] = float("-inf")
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    _say(f"attention all -inf row causal={causal} exact={exact}")
    out, lse, _ = A._launch(q.to(dev), k.to(dev), v.to(dev), None, causal, True, -1 if exact else 13)
    got, lse = out.cpu().float(), lse.cpu()
    assert torch.isnan(got[0, 1, 150]).all()
    assert lse[0, 1, 150] == float("-inf")
    want = R.attention_reference(q, k, v, causal=causal).float()
    keep = torch.ones(B, H, S, dtype=torch.bool)
    keep[0, 1, 150] = False
    torch.testing.assert_close(got[keep], want[keep], rtol=1.6e-2, atol=1e-3)
    torch.testing.assert_close(lse[keep], _lse_reference(q, k, causal)[keep], rtol=LSE_RTOL, atol=LSE_ATOL)


@pytest.mark.parametrize("D,sq,sk,causal", [(64, 200, 90001, False), (256, 130, 70001, False),
                                             (64, 4500, 4500, True), (256, 2100, 2100, True)])
def test_attention_long_key_ranges_other_head_dims(D, sq, sk, causal):
    """Head dims 64 and 256 over more than a thousand key tiles (ragged last tile) and over
    long causal folds, against the fp32 closed form computed on the GPU."""
    dev = _dev()
    g = torch.Generator().manual_seed(21)
    q = torch.randn(1, 1, sq, D, generator=g).bfloat16().to(dev)
    k, v = (torch.randn(1, 1, sk, D, generator=g).bfloat16().to(dev) for _ in range(2))
    _say(f"attention long keys D={D} Sq={sq} Sk={sk} causal={causal}")
    got, lse = CG.run_attention(q, k, v, causal=causal, return_lse=True)
    s = torch.matmul(q.float(), k.float().transpose(-1, -2).contiguous()) / math.sqrt(D)
    if causal:
        s = s.masked_fill(~torch.ones(sq, sk, dtype=torch.bool, device=dev).tril(0),
                          float("-inf"))
    want = torch.matmul(torch.softmax(s, -1), v.float())
    torch.testing.assert_close(got.float(), want, rtol=1.6e-2, atol=1e-3)
    torch.testing.assert_close(lse, torch.logsumexp(s, -1), rtol=LSE_RTOL, atol=LSE_ATOL)


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


def test_attention_graph_replays_match_eager_and_launch_two_kernels():
    """run_attention is the V^T pack and the fold, nothing else (no fill, no assert, no
    synchronisation), so it captures into a HIP graph.  Replays with other eager work between
    them give the eager result every time, also for a block that takes the exact path."""
    from neptune_codegen import hip as H

    dev = _dev()
    g = torch.Generator().manual_seed(19)
    q, k, v = (torch.randn(1, 3, 300, 128, generator=g).bfloat16().to(dev) for _ in range(3))
    v[0, 2, 260, 1] = float("inf")            # head 2, query block 1: exact path
    with H.recording() as rec:
        want, want_lse = CG.run_attention(q, k, v, causal=True, return_lse=True)
    assert len(rec.launches) == 2
    torch.cuda.synchronize()
    _say("attention graph capture, 3 replays")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            out, lse = CG.run_attention(q, k, v, causal=True, return_lse=True)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        out.zero_()
        lse.zero_()
        graph.replay()
        torch.randn(1000, device=dev).sum()   # unrelated eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(torch.isnan(out), torch.isnan(want)), i
        assert torch.equal(out.nan_to_num(0.0, 1.0, -1.0), want.nan_to_num(0.0, 1.0, -1.0)), i
        assert torch.equal(lse, want_lse), i
