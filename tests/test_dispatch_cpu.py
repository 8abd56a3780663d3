"""CPU tests of the launch-plan machinery behind the C++ dispatcher kernels: kernarg image
layout, the recorder, plan extraction, and the operators' registrations."""
import ctypes

import pytest
import torch

from neptune_codegen import dispatch, hip, torch_op


def _kernel(argtypes):
    return hip.Kernel(0, "probe", tuple(argtypes), 64)


@pytest.mark.parametrize("argtypes", [
    (hip.PTR, hip.PTR, hip.I64, hip.I64, hip.I64, hip.I64),
    (hip.PTR,) * 3 + (hip.I32,) * 2 + (hip.I64,) * 3,
    (hip.PTR,) * 6 + (hip.I32,) * 3 + (hip.I64,) * 6 + (hip.F32,),
    (hip.I32, hip.PTR, hip.F32, hip.PTR, hip.I32, hip.I64, hip.PTR),
])
def test_image_layout_is_c_struct_layout(argtypes):
    """Field offsets and packed bytes agree with ctypes' C struct layout of the same list."""
    fields = [(f"a{i}", t) for i, t in enumerate(argtypes)]
    layout = type("Args", (ctypes.Structure,), {"_fields_": fields})
    k = _kernel(argtypes)
    values = [(i + 1) * 0x1000 + 8 if t is hip.PTR else (1.5 * i if t is hip.F32 else 3 * i - 7)
              for i, t in enumerate(argtypes)]
    for i, offset in k.pointer_offsets.items():
        assert offset == getattr(layout, f"a{i}").offset
    assert set(k.pointer_offsets) == {i for i, t in enumerate(argtypes) if t is hip.PTR}
    image = k._packer.pack(*values)
    ref = bytes(layout(*values))
    assert image == ref[:len(image)]
    assert len(ref) - len(image) < 8          # only trailing padding differs


def test_out_of_range_argument_raises():
    """A value that does not fit its parameter raises before anything is launched."""
    k = _kernel((hip.PTR, hip.I32))
    with pytest.raises(ValueError, match="out of range"):
        k.launch((1,), (0, 1 << 40), 0)


def _recorded(launches, buffers=()):
    rec = hip.Recorder()
    rec.launches.extend(launches)
    rec.buffers.extend(buffers)
    return rec


def test_plan_maps_pointers_to_inputs_and_buffers():
    k = _kernel((hip.PTR, hip.PTR, hip.PTR, hip.I64))
    x = torch.randn(4, 8)
    out = torch.empty(4)
    scratch = torch.empty(4, 2)
    args = (x.data_ptr(), out.data_ptr(), scratch.data_ptr(), 4)
    rec = _recorded([(k, (3, 1, 1), k._packer.pack(*args), args)], [scratch])
    buffers, launches = dispatch.plan_of(rec, (x,), (out,))
    code = dispatch.extension().dtype_code
    assert buffers == ((code(out), (4,), (1,)), (code(scratch), (4, 2), (2, 1)))
    assert not any(isinstance(v, torch.Tensor) for b in buffers for v in b)   # metadata only
    handle, grid, block, lds, image, patches = launches[0]
    assert grid == (3, 1, 1) and block == 64
    assert patches == ((0, 0), (8, -1), (16, -2))


def test_plan_refuses_unknown_or_aliased_pointers():
    k = _kernel((hip.PTR, hip.PTR))
    x = torch.randn(4, 8)
    out = torch.empty(4)
    copy = x.clone()
    args = (copy.data_ptr(), out.data_ptr())
    assert dispatch.plan_of(_recorded([(k, (1, 1, 1), k._packer.pack(*args), args)]), (x,), (out,)) is None
    args = (x.data_ptr(), out.data_ptr())
    rec = _recorded([(k, (1, 1, 1), k._packer.pack(*args), args)])
    assert dispatch.plan_of(rec, (x, x[0]), (out,)) is None      # inputs share an address
    assert dispatch.plan_of(rec, (x,), (x,)) is None             # output aliases an input
    null = (x.data_ptr(), 0)
    buffers, launches = dispatch.plan_of(_recorded([(k, (1, 1, 1), k._packer.pack(*null), null)]),
                                         (x,), (out,))
    assert launches[0][5] == ((0, 0),)                           # a null pointer stays literal


def test_recorder_is_scoped_and_thread_local():
    t = torch.empty(2)
    assert hip.scratch(t) is t
    with hip.recording() as outer:
        hip.scratch(t)
        with hip.recording() as inner:
            hip.scratch(t)
        assert len(inner.buffers) == 1
    assert len(outer.buffers) == 1


def test_operators_get_cpp_kernels():
    for overload, n in ((torch_op.op_handle("logsumexp"), 1),
                        (torch_op.op_handle("logsumexp", plan="split"), 1),
                        (torch_op.state_op_handle("rms_norm", {"eps": 1e-5}), 2),
                        (torch_op.state_op_handle("l2_normalize", {"eps": 1e-6}), 1)):
        name = overload._schema.name
        dump = torch._C._dispatch_dump(name)
        assert "CUDA: registered at" in dump and "nep_dispatch.cpp" in dump, dump
        assert "AutogradCUDA: registered at" in dump
        assert set(dispatch.stats(name)) == {"replays", "python_calls", "plans"}
    # CPU tensors still reach the Python body and its refusal
    with pytest.raises(ValueError, match="ROCm"):
        torch_op.op_handle("logsumexp")(torch.randn(2, 8))


def _cpu_op(tag, body, schema="(Tensor x) -> Tensor", n_inputs=1):
    """A custom op whose C++ kernels sit on the CPU keys (bodies allocate, launch nothing)."""
    qualname = f"neptune_dispatch_test::{tag}"
    op = torch.library.custom_op(qualname, mutates_args=(), schema=schema)(body)
    op.register_fake(lambda x, *rest: torch.empty(x.shape[:-1], dtype=x.dtype, device=x.device))
    dispatch.install(qualname, n_inputs, body, backend="CPU")
    return getattr(torch.ops.neptune_dispatch_test, tag).default, qualname


def _rows_body(x, *rest):
    if x.dtype == torch.int32:
        raise TypeError("int32 input refused")
    return torch.empty(x.shape[:-1], dtype=x.dtype, device=x.device)


def test_cpu_backend_records_once_then_replays():
    op, name = _cpu_op("rows", _rows_body)
    x = torch.randn(5, 7)
    a, b, c = op(x), op(x), op(torch.randn(5, 7))
    assert dispatch.stats(name) == {"replays": 2, "python_calls": 1, "plans": 1}
    assert b.shape == (5,) and b.dtype == x.dtype and b.data_ptr() not in (a.data_ptr(), 0)
    op(torch.randn(3, 7))                    # new shape: a new plan
    op(torch.randn(7, 5).t())                # new strides: a new plan
    op(torch.randn(5, 7, dtype=torch.float64))
    assert dispatch.stats(name) == {"replays": 2, "python_calls": 4, "plans": 4}
    with pytest.raises(TypeError, match="int32 input refused"):
        op(torch.ones(2, 3, dtype=torch.int32))
    dispatch.clear()                         # (a refused call counts nothing)
    op(x)
    assert dispatch.stats(name) == {"replays": 2, "python_calls": 5, "plans": 5}


def test_cpu_backend_aliased_inputs_stay_in_python():
    op, name = _cpu_op("pair", _rows_body, "(Tensor x, Tensor g) -> Tensor", 2)
    x = torch.randn(4, 6)
    op(x, x[0])
    op(x, x[0])
    assert dispatch.stats(name) == {"replays": 0, "python_calls": 2, "plans": 0}
    g = torch.randn(6)
    op(x, g)
    op(x, g)
    assert dispatch.stats(name) == {"replays": 1, "python_calls": 3, "plans": 1}


def test_cpu_backend_grad_goes_through_the_original_autograd_kernel():
    op, name = _cpu_op("graded", _rows_body)
    x = torch.randn(4, 6, requires_grad=True)
    out = op(x)
    assert out.requires_grad and out.grad_fn is not None
    with pytest.raises(RuntimeError, match="autograd"):
        out.sum().backward()
    with torch.no_grad():
        assert not op(x).requires_grad
    assert dispatch.stats(name)["replays"] == 1


# ---------------------------------------------------------------- launch-plan bundles
import struct  # noqa: E402


def _bundle(ops, codes=()):
    """Bytes of a bundle in libneptune_ops' format (see nep_ops.cpp)."""
    def s(text):
        data = text.encode()
        return struct.pack("<I", len(data)) + data

    blob = b"NEPBNDL1" + struct.pack("<I", len(codes))
    for code in codes:
        blob += struct.pack("<I", len(code)) + code
    blob += struct.pack("<I", len(ops))
    for qualname, arguments, n_inputs, plans in ops:
        blob += s(qualname) + s(arguments) + struct.pack("<II", n_inputs, len(plans))
        for key, buffers in plans:
            blob += struct.pack("<I", len(key)) + struct.pack(f"<{len(key)}q", *key)
            blob += struct.pack("<I", len(buffers))
            for code, sizes, strides in buffers:
                blob += struct.pack("<iI", code, len(sizes)) + struct.pack(f"<{len(sizes)}q", *sizes)
                blob += struct.pack(f"<{len(strides)}q", *strides)
            blob += struct.pack("<I", 0)                 # no launches
    return blob


def _load_ops_library():
    torch.ops.load_library(str(dispatch.OPS_LIBRARY))
    return torch.ops.neptune_bundle.load


def test_bundle_loader_defines_operators_once(tmp_path):
    load = _load_ops_library()
    path = tmp_path / "ok.nepb"
    plan = ([6, 0, 2, 4, 8, 8, 1, 0], [(6, [4], [1])])
    path.write_bytes(_bundle([("neptune_bundle_test::rows", "(Tensor x) -> Tensor", 1, [plan])]))
    assert load(str(path)) == 1
    dump = torch._C._dispatch_dump("neptune_bundle_test::rows")
    assert "CUDA: registered at" in dump and "nep_ops.cpp" in dump, dump
    assert str(torch._C._get_schema("neptune_bundle_test::rows", "")).endswith("(Tensor x) -> Tensor")
    assert load(str(path)) == 0                          # already defined: left as it is


@pytest.mark.parametrize("mutate, needle", [
    (lambda b: b"NOTABNDL" + b[8:], "bad magic"),
    (lambda b: b[:-5], "truncated"),
    (lambda b: b + b"\0", "trailing"),
])
def test_bundle_loader_refuses_damaged_files(tmp_path, mutate, needle):
    load = _load_ops_library()
    good = _bundle([("neptune_bundle_test::damaged", "(Tensor x) -> Tensor", 1,
                     [([6, 0, 1, 4, 1, 0], [(6, [], [])])])])
    path = tmp_path / "bad.nepb"
    path.write_bytes(mutate(good))
    with pytest.raises(RuntimeError, match=needle):
        load(str(path))


def test_export_bundle_needs_recorded_plans(tmp_path):
    op = torch_op.op_handle("logsumexp")
    with pytest.raises(ValueError, match="no recorded launch plan"):
        dispatch.export_bundle(tmp_path / "x.nepb", [op._schema.name + "_never_run"])


def test_cpu_backend_caps_plans_per_operator():
    op, name = _cpu_op("capped", _rows_body)
    for n in range(1, dispatch.MAX_PLANS + 1):
        op(torch.empty(n, 3))
    assert dispatch.stats(name)["plans"] == dispatch.MAX_PLANS
    extra = torch.empty(dispatch.MAX_PLANS + 7, 3)
    op(extra)
    op(extra)
    s = dispatch.stats(name)
    assert s["plans"] == dispatch.MAX_PLANS and s["replays"] == 0
    assert s["python_calls"] == dispatch.MAX_PLANS + 2
    op(torch.empty(1, 3))                                   # an early layout still replays
    assert dispatch.stats(name)["replays"] == 1
