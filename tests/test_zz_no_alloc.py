"""nep_fold_split_noalloc: the split plan with the library's own per-GPU scratch array.

Called through the C ABI and checked bit for bit against nep_fold_split (the same kernels over
a caller workspace) on two calls in a row, the second on a smaller input, so a stale partial
left by the first call in the shared array would show; a request above the array's capacity
is refused before any launch.
"""
import ctypes

import pytest
import torch

from neptune_codegen import hip
from tests.test_gpu_split_abi import run_entry, split_call

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda:0")


def run_noalloc(x, block=1024, name="logsumexp"):
    lib = hip.load_library()
    kp, km, rows, ncols, nparts, threads, ppw = split_call(x, name, block)
    out = torch.empty(rows, dtype=x.dtype, device=x.device)
    rc = lib.nep_fold_split_noalloc(kp.handle, km.handle, ctypes.c_void_p(x.data_ptr()),
                                    ctypes.c_void_p(out.data_ptr()), rows, ncols, x.stride(0),
                                    x.stride(1), nparts, block, threads, ppw,
                                    ctypes.c_void_p(hip.current_stream(x.device)))
    assert rc == 0, lib.nep_last_error()
    return out


def _same_bits(a, b):
    assert torch.equal(torch.isnan(a), torch.isnan(b))
    view = torch.int16 if a.element_size() == 2 else torch.int32
    assert torch.equal(a.nan_to_num(0.0).view(view), b.nan_to_num(0.0).view(view))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_split_matches_the_workspace_entry_point_twice(dtype):
    dev = _dev()
    g = torch.Generator().manual_seed(31)
    big = (4 * torch.randn(64, 262144, generator=g)).to(dtype).to(dev)   # 16384 partials
    small = (4 * torch.randn(5, 3000, generator=g)).to(dtype).to(dev)    # 15 partials
    small[2, 7] = float("inf")
    for x in (big, small):
        print(f"noalloc split {dtype} {tuple(x.shape)}", flush=True)
        got = run_noalloc(x)
        want = run_entry(x)
        torch.cuda.synchronize()
        _same_bits(got, want)


def test_noalloc_split_refuses_more_than_its_scratch():
    lib = hip.load_library()
    capacity = lib.nep_fold_split_noalloc_capacity()
    assert capacity == 8 << 20
    rows, nparts, block = capacity // 16 // 4096 + 1, 4096, 64      # one row too many
    ncols = nparts * block
    rc = lib.nep_fold_split_noalloc(1, 1, ctypes.c_void_p(16), ctypes.c_void_p(16), rows, ncols,
                                    ncols, 1, nparts, block, 256, 4, None)
    assert rc == 1
    assert b"more than the 8388608 bytes" in lib.nep_last_error()
