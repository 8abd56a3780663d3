"""Exhaustive GPU check of nep::bf16x2_rne (the hardware fp32 -> bf16 conversion
v_cvt_pk_bf16_f32) against the integer round-to-nearest-even nep::f32_to_bf16_bits, over all
2^32 fp32 bit patterns.

The storage path of every bf16 fold may use the hardware conversion only because this test
shows it bit-identical to the integer rounding for every non-NaN input (ties, denormals,
overflow to inf, infinities) and NaN-preserving for NaN inputs.  Each workgroup counts its
mismatches with ballots and writes one count (plain stores, no atomics)."""
import pytest
import torch

from neptune_codegen import hip
from neptune_codegen.emitters import BASE_OPTIONS, kernel_header

pytestmark = pytest.mark.gpu

PER_THREAD = 64
BLOCK = 256

SRC = kernel_header("nep_device.h") + r'''
extern "C" __global__ void __launch_bounds__(256) bf16_conversion_check(unsigned* counts) {
  const unsigned base = (blockIdx.x * 256u + threadIdx.x) * 64u;
  unsigned bad = 0, bad_nan = 0;
  for (unsigned i = 0; i < 64u; i += 2) {
    const unsigned b0 = base + i, b1 = base + i + 1;
    const float f0 = nep::as_f32(b0), f1 = nep::as_f32(b1);
    const unsigned hw = nep::bf16x2_rne(f0, f1);
    const unsigned h0 = hw & 0xffffu, h1 = hw >> 16;
    const unsigned s0 = nep::f32_to_bf16_bits(f0), s1 = nep::f32_to_bf16_bits(f1);
    if (f0 == f0) bad += h0 != s0; else bad_nan += (h0 & 0x7fffu) <= 0x7f80u;
    if (f1 == f1) bad += h1 != s1; else bad_nan += (h1 & 0x7fffu) <= 0x7f80u;
  }
  // block totals: wave sums through the LDS, one plain store per block
  __shared__ unsigned part[2][4];
  unsigned w0 = bad, w1 = bad_nan;
  w0 += nep::partner_u32<1>(w0); w1 += nep::partner_u32<1>(w1);
  w0 += nep::partner_u32<2>(w0); w1 += nep::partner_u32<2>(w1);
  w0 += nep::partner_u32<4>(w0); w1 += nep::partner_u32<4>(w1);
  w0 += nep::partner_u32<8>(w0); w1 += nep::partner_u32<8>(w1);
  w0 += nep::partner_u32<16>(w0); w1 += nep::partner_u32<16>(w1);
  w0 += nep::partner_u32<32>(w0); w1 += nep::partner_u32<32>(w1);
  if ((threadIdx.x & 63) == 0) { part[0][threadIdx.x >> 6] = w0; part[1][threadIdx.x >> 6] = w1; }
  __syncthreads();
  if (threadIdx.x == 0) {
    counts[2 * blockIdx.x] = part[0][0] + part[0][1] + part[0][2] + part[0][3];
    counts[2 * blockIdx.x + 1] = part[1][0] + part[1][1] + part[1][2] + part[1][3];
  }
}
'''


def test_hw_bf16_conversion_is_integer_rtne_for_all_fp32_patterns():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    dev = torch.device("cuda:0")
    blocks = (1 << 32) // (BLOCK * PER_THREAD)
    counts = torch.zeros(2 * blocks, dtype=torch.int32, device=dev)
    k = hip.Program(SRC, "bf16_conversion_check.hip", BASE_OPTIONS).kernel(
        "bf16_conversion_check", (hip.PTR,), BLOCK, 0)
    print(f"bf16 conversion check: {blocks} blocks x {BLOCK * PER_THREAD} patterns", flush=True)
    k.launch((blocks,), (counts.data_ptr(),), hip.current_stream(dev))
    c = counts.view(blocks, 2).to(torch.int64).sum(0).cpu()
    assert int(c[0]) == 0, f"{int(c[0])} non-NaN inputs round differently"
    assert int(c[1]) == 0, f"{int(c[1])} NaN inputs did not stay NaN"
