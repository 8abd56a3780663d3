"""GPU tests at sizes past 2^31 elements: every kernel indexes with 64-bit offsets, so the
rows and segments that sit beyond the 32-bit element range must come out exactly as the same
rows computed alone (and as the oracle says).  Inputs are generated on the device; only the
checked rows are copied back."""
import pytest
import torch

import neptune_codegen as CG
from oracle import references as R

pytestmark = pytest.mark.gpu

ROWS, COLS = 65600, 32768          # 2 149 580 800 elements (> 2^31), 4.3 GB in bf16


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda:0")


def _big(dev, dtype=torch.bfloat16, scale=4.0, seed=51):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.empty(ROWS, COLS, dtype=dtype, device=dev)
    for i in range(0, ROWS, 8192):          # in slabs: keeps the fp32 temporary small
        x[i:i + 8192] = (scale * torch.randn(min(8192, ROWS - i), COLS, generator=g, device=dev)).to(dtype)
    assert x.numel() > 2 ** 31
    return x


CHECK = (0, 1, 32767, 65535, 65536, ROWS - 1)      # rows on both sides of the 2^31 boundary


def test_logsumexp_and_readout_past_2_pow_31_elements():
    dev = _dev()
    x = _big(dev)
    print(f"logsumexp bf16 [{ROWS},{COLS}]", flush=True)
    got = CG.run("logsumexp", x)
    torch.cuda.synchronize()
    rows = x[list(CHECK)].cpu()
    want = R.reference("logsumexp", rows)
    torch.testing.assert_close(got[list(CHECK)].cpu().float(), want.to(torch.bfloat16).float(),
                               rtol=1.6e-2, atol=1e-3)
    alone = CG.run("logsumexp", x[list(CHECK)].contiguous())
    assert torch.equal(got[list(CHECK)], alone)
    print(f"log_softmax readout bf16 [{ROWS},{COLS}]", flush=True)
    out = CG.run_log_softmax(x)
    torch.cuda.synchronize()
    part = out[list(CHECK)].cpu().float()
    ref = torch.log_softmax(rows.float(), -1).to(torch.bfloat16).float()
    torch.testing.assert_close(part, ref, rtol=1.6e-2, atol=1e-3)
    del out


def test_rms_norm_past_2_pow_31_elements():
    dev = _dev()
    x = _big(dev, scale=1.0, seed=52)
    gamma = (1 + 0.1 * torch.randn(COLS, generator=torch.Generator().manual_seed(53))).bfloat16()
    print(f"rms_norm bf16 [{ROWS},{COLS}]", flush=True)
    got = CG.run_rms_norm(x, gamma.to(dev), eps=1e-6)
    torch.cuda.synchronize()
    rows = x[list(CHECK)].cpu()
    want = R.rms_norm_reference(rows, gamma, 1e-6).float()
    torch.testing.assert_close(got[list(CHECK)].cpu().float(), want, rtol=1.6e-2, atol=1e-3)


def test_segment_sum_past_2_pow_31_elements():
    """128-token segments over 2^24 + 4096 tokens of 128 fp16 channels: the last segments start
    past element 2^31 and must be bit-exact against the ordered oracle."""
    dev = _dev()
    tokens = (1 << 24) + 4096
    g = torch.Generator(device=dev).manual_seed(54)
    data = torch.randn(tokens, 128, generator=g, device=dev).half()
    lengths = torch.full((tokens // 128,), 128, dtype=torch.int64)
    print(f"segment_sum fp16 [{tokens},128], {lengths.numel()} segments", flush=True)
    got = CG.run_segment_pool(data, lengths.to(dev), reduce="sum")
    torch.cuda.synchronize()
    for seg in (0, 1, lengths.numel() // 2, lengths.numel() - 2, lengths.numel() - 1):
        part = data[seg * 128:(seg + 1) * 128].cpu()
        want = R.segment_reference(part, torch.tensor([128], dtype=torch.int32), "sum")
        assert torch.equal(got[seg:seg + 1].cpu(), want), seg
