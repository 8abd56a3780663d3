"""The C-ABI library: loads, exports every function include/neptune_hip.h declares, compiles
for gfx950 through hiprtc without a GPU, and reports errors through nep_last_error.
No compute call is made here (no GPU on the CPU runner)."""
import ctypes
import pathlib
import re

import pytest

from neptune_codegen import hip

HEADER = pathlib.Path(__file__).resolve().parent.parent / "include" / "neptune_hip.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(nep_\w+)\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = hip.load_library()
    names = declared()
    assert set(names) == set(hip.EXPORTED), names
    for name in names:
        assert getattr(lib, name) is not None
    assert lib.nep_abi_version() == 2


def test_ops_library_exports_its_declared_symbol(tmp_path):
    """libneptune_ops.so exports what include/neptune_ops.h declares; the C entry point reports
    a damaged bundle through its error buffer (no GPU is touched before the magic check)."""
    from neptune_codegen import dispatch

    header = HEADER.parent / "neptune_ops.h"
    names = sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(nep_\w+)\(", header.read_text(), re.M)))
    assert names == ["nep_ops_load_bundle"]
    import torch  # noqa: F401 -- the library resolves against torch's libraries

    lib = ctypes.CDLL(str(dispatch.OPS_LIBRARY))
    fn = lib.nep_ops_load_bundle
    fn.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
    fn.restype = ctypes.c_int
    bad = tmp_path / "bad.nepb"
    bad.write_bytes(b"not a bundle at all")
    err = ctypes.create_string_buffer(256)
    assert fn(str(bad).encode(), err, len(err)) == -1
    assert b"bad magic" in err.value
    assert fn(str(tmp_path / "missing.nepb").encode(), err, len(err)) == -1
    assert b"cannot open" in err.value


def test_compile_code_object_and_error_reporting():
    lib = hip.load_library()
    ok = 'extern "C" __global__ void k(float* x) { x[threadIdx.x] *= 2.0f; }'
    assert hip.compile_code_object(ok, "ok.hip", ("--offload-arch=gfx950", "-O3"), write_cache=False) > 0
    with pytest.raises(hip.HipError, match="hiprtc compile"):
        hip.compile_code_object("this is not C++", "bad.hip", ("--offload-arch=gfx950",), write_cache=False)
    assert b"bad.hip" in lib.nep_last_error()


def test_argument_checks_need_no_gpu():
    lib = hip.load_library()
    grid = (ctypes.c_uint32 * 3)(1, 1, 1)
    block = (ctypes.c_uint32 * 3)(64, 1, 1)
    assert lib.nep_launch(0, grid, block, 0, None, None, 0) == 1          # NEP_ERR_INVALID
    assert b"null kernel" in lib.nep_last_error()
    out = ctypes.c_uint64()
    assert lib.nep_get_kernel(0, b"k", ctypes.byref(out)) == 1
    assert lib.nep_compile(None, b"x", b"", None, ctypes.byref(out)) == 1


def test_split_entry_point_checks_its_arguments_before_any_launch():
    """nep_fold_split refuses inconsistent shapes (no GPU is touched before the checks)."""
    lib = hip.load_library()
    ws = ctypes.c_void_p(16)
    common = dict(x=ctypes.c_void_p(16), out=ctypes.c_void_p(16))

    def call(partial=1, merge=1, rows=4, ncols=3000, nparts=3, block=1024, threads=256, ppw=4,
             workspace=ws, nbytes=1 << 20):
        return lib.nep_fold_split(partial, merge, common["x"], common["out"], rows, ncols, ncols, 1,
                                  nparts, block, threads, ppw, workspace, nbytes, None)

    assert lib.nep_fold_split_workspace_bytes(64, 256) == 16 * 64 * 256
    assert lib.nep_fold_split_workspace_bytes(0, 256) == 0
    for kwargs, needle in (({"partial": 0}, b"null kernel"), ({"nparts": 2}, b"ceil(ncols / block)"),
                           ({"block": 1000, "nparts": 3}, b"power of two"),
                           ({"ncols": 5000 * 1024, "nparts": 5000}, b"capacity"),
                           ({"threads": 100}, b"multiple of 64"), ({"ppw": 0}, b"parts_per_workgroup"),
                           ({"nbytes": 100}, b"workspace holds 100 bytes"),
                           ({"workspace": None}, b"workspace")):
        assert call(**kwargs) == 1, kwargs
        assert needle in lib.nep_last_error(), (kwargs, lib.nep_last_error())
    assert call(rows=0) == 0            # nothing to do, nothing launched
