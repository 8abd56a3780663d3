"""The typed split entry point of the C ABI (nep_fold_split) on the GPU.

It runs the same generated partial / merge kernels as the Python split path, so its results
must be bit-identical to CG.run(..., plan="split"), which is itself checked against the oracle
(tests/test_gpu_folds.py).  Called through ctypes with a torch-allocated workspace.
"""
import ctypes

import pytest
import torch

import neptune_codegen as CG
from neptune_codegen import hip
from neptune_codegen import template as T

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch.device("cuda:0")


def split_call(x, name="logsumexp", block=1024, **params):
    """(kernel handles and launch numbers) the product's split path picks for x (2-D)."""
    params = {**CG.param_defaults(name), **params}
    partial, merge = CG.compile_skeleton(name, params, plan="split")
    rows, ncols = x.shape
    nparts, _ = CG.split_launch_shape(ncols, block)
    var = T._fold_variant(x, ncols, block, 4, split_block=block)
    device = x.device.index or 0
    kp = partial.kernel(var, "partial", device)
    km = merge.kernel(var, "merge", device)
    return kp, km, rows, ncols, nparts, var.wg, max(1, var.wg // var.tpr)


def run_entry(x, block=1024, name="logsumexp", threads=None, ppw=None, expect_rc=0, **params):
    lib = hip.load_library()
    kp, km, rows, ncols, nparts, wg, rpw = split_call(x, name, block, **params)
    threads = wg if threads is None else threads
    ppw = rpw if ppw is None else ppw
    out = torch.empty(rows, dtype=x.dtype, device=x.device)
    nbytes = lib.nep_fold_split_workspace_bytes(rows, nparts)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    rc = lib.nep_fold_split(kp.handle, km.handle, ctypes.c_void_p(x.data_ptr()),
                            ctypes.c_void_p(out.data_ptr()), rows, ncols, x.stride(0), x.stride(1),
                            nparts, block, threads, ppw, ctypes.c_void_p(ws.data_ptr()), nbytes,
                            ctypes.c_void_p(hip.current_stream(x.device)))
    assert rc == expect_rc, lib.nep_last_error()
    return out


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape,block", [((64, 262144), 1024), ((7, 5000), 256), ((3, 1), 1024),
                                         ((33, 1025), 1024)])
def test_split_entry_point_matches_the_python_split_path(dtype, shape, block):
    dev = _dev()
    g = torch.Generator().manual_seed(21)
    x = (4 * torch.randn(*shape, generator=g)).to(dtype).to(dev)
    if shape[1] > 10:
        x[0, 3] = float("inf")
        x[1, 5] = float("nan")
    print(f"nep_fold_split {dtype} {shape} block {block}", flush=True)
    got = run_entry(x, block)
    want = CG.run("logsumexp", x, plan="split", block=block)
    torch.cuda.synchronize()
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    assert torch.equal(_bits(got.nan_to_num(0.0)), _bits(want.nan_to_num(0.0)))


def test_split_entry_point_strided_rows_and_another_skeleton():
    dev = _dev()
    g = torch.Generator().manual_seed(22)
    base = torch.randn(16, 9000, generator=g).abs().add(0.1).to(dev)
    x = base[::2, 100:8100]                         # row stride 18000, offset start
    print("nep_fold_split stable_l2 strided", flush=True)
    got = run_entry(x, 512, "stable_l2")
    want = CG.run("stable_l2", x, plan="split", block=512)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_split_entry_point_checks_the_launch_numbers_against_the_kernel():
    """partial_threads and parts_per_workgroup are checked against what the generated unit
    holds (the partial kernel's workgroup bound, and the size of its parts-per-workgroup marker
    symbol): any other value fails with NEP_ERR_INVALID before any launch, while the kernel's
    own numbers give the Python split path's result."""
    dev = _dev()
    g = torch.Generator().manual_seed(23)
    x = (4 * torch.randn(48, 20000, generator=g)).bfloat16().to(dev)
    want = CG.run("logsumexp", x, plan="split", block=1024)
    _, _, _, _, _, wg, rpw = split_call(x, "logsumexp", 1024)
    lib = hip.load_library()
    for threads in sorted({64, 128, 256, 512, 1024} - {wg}):
        print(f"nep_fold_split refuses partial_threads={threads} (kernel: {wg})", flush=True)
        run_entry(x, 1024, threads=threads, expect_rc=1)
        assert b"workgroup size" in lib.nep_last_error()
    for ppw in sorted({1, max(1, rpw // 2), min(wg, 2 * rpw), min(wg, 8 * rpw)} - {rpw}):
        print(f"nep_fold_split refuses parts_per_workgroup={ppw} (kernel: {rpw})", flush=True)
        run_entry(x, 1024, ppw=ppw, expect_rc=1)
        assert b"parts_per_workgroup" in lib.nep_last_error()
    got = run_entry(x, 1024)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(want))
