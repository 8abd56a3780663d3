"""The operator bridge without a GPU: refusal semantics, metadata, operator identity and the
launch ABI (recorded, not executed).  Mirrors the reference's tests/test_autotune.py:424-505,
625-749, 1028-1150 and tests/test_neptune_opt.py:957-970, 1034-1065 for the HIP backend.
"""
import json
import pathlib

import pytest
import torch

import neptune_codegen as CG
from neptune_codegen import autotune, hip
from neptune_codegen import template as T
from neptune_codegen import torch_op as TO

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def meta(shape, dtype=torch.float32):
    return torch.empty(shape, device="meta", dtype=dtype)


def test_row_last_refusals_and_metadata_shapes():
    cases = [(torch.empty(2, 8), ValueError, "device"),
             (meta(()), ValueError, "rank"),
             (meta((2, 0)), RuntimeError, "width"),
             (meta((2, 8), torch.float64), TypeError, "dtype"),
             (meta((2, 8), torch.int32), TypeError, "dtype")]
    for x, error, message in cases:
        with pytest.raises(error, match=message):
            CG.run("logsumexp", x)
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        for shape in ((8,), (2, 3, 8), (2, 0, 8)):
            for keep in (False, True):
                for plan in ("serial", "split"):
                    out = CG.run("logsumexp", meta(shape, dtype), keepdim=keep, plan=plan)
                    assert out.shape == shape[:-1] + ((1,) if keep else ())
                    assert out.dtype == dtype


def test_split_capacity_golden():
    table = json.loads((GOLDEN / "split_capacity.json").read_text())
    for ncols, block, nparts, width in table["ok"]:
        assert CG.split_launch_shape(ncols, block) == (nparts, width)
    for case in table["refused"]:
        error = {"NotImplementedError": NotImplementedError, "ValueError": ValueError}[case["error"]]
        with pytest.raises(error, match=case["match"]):
            CG.split_launch_shape(case["ncols"], case["block"])

    class Symbolic:
        def __int__(self):
            raise AssertionError("must not concretise")

    with pytest.raises(NotImplementedError, match="concrete width"):
        CG.split_launch_shape(Symbolic(), 1024)


def test_two_pass_folds_refuse_the_split_plan():
    """variance and std carry (mean, M2) over a second pass; the pair merge a split needs is
    refused for them and the other skeletons compile a split pair."""
    for name, sk in CG.SKELETONS.items():
        if sk.two_pass:
            with pytest.raises(NotImplementedError, match="two_pass needs extended carried state"):
                CG.compile_skeleton(name, CG.param_defaults(name), plan="split")
        else:
            assert len(CG.compile_skeleton(name, CG.param_defaults(name), plan="split")) == 2


def test_split_certificate_and_structured_programs_are_reused_per_parameter_set():
    """The merge certificate (a symbolic proof, ~1 ms) and the structured program are kept per
    exact parameter set: a repeated call gets the same object, a value of another type or sign
    is proved and validated afresh, and refusals are raised every time."""
    from neptune_codegen.algebra import derive_merge_certificate

    sk = CG.SKELETONS["softcap_lse"]
    a = derive_merge_certificate(sk, {"beta": 1.0, "tiny": 0.0})
    assert derive_merge_certificate(sk, {"tiny": 0.0, "beta": 1.0}) is a
    assert derive_merge_certificate(sk, {"beta": 1.0, "tiny": -0.0}) is not a
    assert derive_merge_certificate(sk, {"beta": 1, "tiny": 0.0}) is not a
    for _ in range(2):
        with pytest.raises(NotImplementedError, match="two_pass"):
            derive_merge_certificate(CG.SKELETONS["variance"], {})
    prog = T.compile_state_reduction("rms_norm", {"eps": 0.5})
    assert T.compile_state_reduction("rms_norm", {"eps": 0.5}) is prog
    for bad in ({"eps": True}, {"eps": "0.5"}, {"eps": 0.0}, {"eps": 0.5, "extra": 1}):
        for _ in range(2):
            with pytest.raises(ValueError):
                T.compile_state_reduction("rms_norm", bad)


def test_operator_identity_golden():
    table = json.loads((GOLDEN / "op_keys.json").read_text())
    for args, want in table["op_key"]:
        assert autotune.op_key(*args) == want
    for name, want in table["machine_key"]:
        assert autotune.machine_key(name) == want
    a = {"alpha": 1.0000001, "beta": 2.0}
    assert autotune.parameter_tag(a) == autotune.parameter_tag(dict(reversed(list(a.items()))))
    assert autotune.parameter_tag({"a": 1, "b": 2}) != autotune.parameter_tag({"a1_b": 2})
    keys = [autotune.op_key("neptune", "softcap_lse", {"beta": v}, False)
            for v in (1.0, 1.0000001, 1.0000002, -0.0, 0.0, 1e-8, 1e8)]
    assert len(set(keys)) == 7 and all(k.split("::")[1].isidentifier() for k in keys)


def test_rms_metadata_validation():
    cases = [(meta(()), meta((1,)), ValueError, "rank"),
             (meta((2, 0)), meta((0,)), RuntimeError, "width"),
             (meta((2, 8), torch.int32), meta((8,), torch.int32), TypeError, "dtype"),
             (meta((2, 8), torch.float16), meta((8,)), ValueError, "dtype/device"),
             (meta((2, 8)), meta((1, 8)), ValueError, "1D"),
             (meta((2, 8)), meta((7,)), RuntimeError, "width"),
             (meta((2, 8)), torch.empty(8), ValueError, "dtype/device")]
    for x, gamma, error, message in cases:
        with pytest.raises(error, match=message):
            CG.run_rms_norm(x, gamma)
    with pytest.raises(ValueError, match="device"):
        CG.run_rms_norm(torch.empty(2, 8), torch.empty(8))
    for width, plan in ((32768, "serial"), (32769, "split"), (4194304, "split")):
        assert CG.validate_rms_inputs(meta((0, width)), meta((width,)), {"eps": 1e-6},
                                      plan=plan, metadata=True) == (0, width)
    for width, plan, message in ((32769, "serial", "32768"), (4194305, "split", "capacity")):
        with pytest.raises(NotImplementedError, match=message):
            CG.validate_rms_inputs(meta((0, width)), meta((width,)), {"eps": 1e-6}, plan=plan, metadata=True)
    for eps in (True, "1e-6", None, 0, -1, float("inf"), float("nan")):
        with pytest.raises(ValueError, match="eps"):
            CG.run_rms_norm(meta((2, 8)), meta((8,)), eps=eps)
    out = CG.run_rms_norm(meta((512, 2)).t(), meta((512,)))
    assert out.stride() == (512, 1)
    assert CG.run_l2_normalize(meta((3, 7), torch.bfloat16)).shape == (3, 7)


def test_segment_metadata_and_span_checks():
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        for shape, count, offsets in (((0,), 0, False), ((3, 0, 2), 2, False), ((0, 2), 1, True),
                                      ((4, 2, 3), 4, True)):
            out = CG.run_segment_pool(meta(shape, dtype), meta((count,), torch.int32), offsets=offsets)
            assert out.shape == ((count - 1 if offsets else count),) + shape[1:] and out.dtype == dtype
    with pytest.raises(RuntimeError, match="boundary"):
        CG.validate_segment_inputs(torch.empty(3), torch.empty(0, dtype=torch.int64), metadata=True, offsets=True)
    for data, segments, error in ((torch.empty(()), torch.empty(2, dtype=torch.int64), ValueError),
                                  (torch.empty(3, dtype=torch.float64), torch.empty(2, dtype=torch.int64), TypeError),
                                  (torch.empty(3), torch.empty(2), TypeError),
                                  (torch.empty(3), torch.empty(2, 1, dtype=torch.int64), ValueError)):
        with pytest.raises(error):
            CG.validate_segment_inputs(data, segments, metadata=True)
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        with pytest.raises(RuntimeError, match="overflow"):
            CG.validate_segment_inputs(torch.empty(3, dtype=dtype), torch.tensor([3]), metadata=True, initial=1e300)
    with pytest.raises(ValueError, match="CUDA"):
        CG.run_segment_pool(torch.empty(3), torch.tensor([3]))
    with pytest.raises(NotImplementedError, match="ordered"):
        CG.run_segment_pool(torch.empty(3), torch.tensor([3]), plan="split")
    with pytest.raises(ValueError, match="finite"):
        CG.compile_segment_reduction("segment_sum", {"initial": float("nan")})
    with pytest.raises(ValueError, match="unknown segment parameters"):
        CG.compile_segment_reduction("segment_sum", {"typo": 1})
    # the prefix construction and the device-side asserts (CPU: raised synchronously)
    x = torch.empty(7, 2)
    spans = TO._segment_spans(x, torch.tensor([0, 2, 0, 5], dtype=torch.int32), offsets=False, unsafe=False)
    assert spans.dtype == torch.int64 and spans.tolist() == [0, 0, 2, 2, 7]
    for indices, is_offsets, unsafe in (([-1, 8], False, False), ([3, 3], False, False), ([8], False, True),
                                        ([4, 4], False, True), ([-1, 4], True, True), ([0, 8], True, False),
                                        ([4, 3], True, True)):
        with pytest.raises(RuntimeError):
            TO._segment_spans(x, torch.tensor(indices), offsets=is_offsets, unsafe=unsafe)


class _Recorder:
    def __init__(self, name):
        self.name, self.calls = name, []

    def launch(self, grid, args, stream):
        self.calls.append((tuple(grid), tuple(args)))


@pytest.fixture
def recorded(monkeypatch):
    """Replaces kernel loading by recorders; the host launch ABI runs for real."""
    made = {}

    def kernel(self, var, stage, device):
        return made.setdefault(stage, _Recorder(stage))

    monkeypatch.setattr(T.FoldProgram, "kernel", kernel)
    monkeypatch.setattr(hip, "current_stream", lambda device: 0)
    monkeypatch.setattr(torch.cuda, "current_device", lambda: 0)
    return made


def test_scalar_launch_abi(recorded):
    base = torch.randn(4, 6, 8)
    inputs = [torch.randn(3, 8), torch.randn(3, 16)[:, ::2], torch.randn(8, 3).t(), base[:, :, ::2],
              base.transpose(0, 1)]
    kernel = CG.compile_skeleton("logsumexp", {"tiny": 0.0})
    for x in inputs:
        x2, rows, ncols = T._row_last_layout(x)
        out = torch.empty(rows)
        T.launch_reduction(kernel, "serial", x2, out, rows, ncols, 1024, 4)
        grid, args = recorded[""].calls[-1]
        assert args == (x2.data_ptr(), out.data_ptr(), rows, ncols, x2.stride(0), x2.stride(1))
        if x.ndim <= 2:
            assert x2.data_ptr() == x.data_ptr(), "a viewable input must not be copied"
    assert T._row_last_layout(inputs[-1])[0].data_ptr() != inputs[-1].data_ptr()


def test_launch_shapes_per_fold_class():
    """fp32 16384 x 4096 at the default (4096, 4): the plain exponential fold keeps 4 slots on
    256 lanes; non-exponential single-pass folds and exponential folds with a transcendental
    producer take 8 slots on 128 lanes (one tile per row either way); two-pass folds keep the
    whole row resident."""
    x = torch.empty(16384, 4096)

    def shape(name):
        sk = CG.SKELETONS[name]
        prog = T.FoldProgram(name, {}, "serial")
        var = T._fold_variant(x, 4096, 4096, 4, resident=sk.two_pass,
                              merge_heavy=not sk.is_log and not sk.two_pass,
                              heavy_phi=prog.heavy_phi)
        return var.tpr, var.unroll, var.tpr * var.unroll * 4

    assert shape("logsumexp") == (256, 4, 4096)
    assert T.FoldProgram("softcap_lse", {}, "serial").heavy_phi
    for name in ("softcap_lse", "rmsnorm_max", "stable_l2"):
        assert shape(name) == (128, 8, 4096), name
    assert shape("variance")[2] >= 4096

    # bf16 rows at the default shape: non-exponential single-pass folds take ~width/128 lanes
    # (16..64) and walk several tiles; two-pass folds become resident through lanes first
    def shape16(name, ncols):
        sk = CG.SKELETONS[name]
        block, warps = autotune.default_config(16384, ncols, torch.bfloat16)[:2]
        var = T._fold_variant(torch.empty(1, ncols, dtype=torch.bfloat16), ncols, block, warps,
                              resident=sk.two_pass, merge_heavy=not sk.is_log and not sk.two_pass)
        return var.tpr, var.unroll

    assert [shape16("rmsnorm_max", n) for n in (1000, 4096, 16384, 32000)] == \
        [(16, 4), (32, 4), (64, 4), (64, 8)]
    assert [shape16("variance", n) for n in (1000, 4096, 16384, 32000)] == \
        [(32, 4), (128, 4), (512, 4), (512, 8)]


def test_split_launch_abi(recorded):
    x = torch.empty((2, 17), dtype=torch.bfloat16)[:, ::2]
    out = torch.empty((2,), dtype=x.dtype)
    kernel = CG.compile_skeleton("stable_l2", {}, plan="split")
    T.launch_reduction(kernel, "split", x, out, 2, 9, 4, 1)
    (pgrid, pargs), (mgrid, margs) = recorded["partial"].calls[-1], recorded["merge"].calls[-1]
    assert pargs[0] == x.data_ptr() and pargs[5:] == (2, 9, x.stride(0), x.stride(1), 3, 4)
    assert margs[:4] == pargs[1:5], "merge reads the partial scratch the partial kernel wrote"
    assert margs[4] == out.data_ptr() and margs[5:] == (2, 9, 3)


def test_custom_op_registration_and_fake_without_gpu():
    from torch._subclasses.fake_tensor import FakeTensorMode

    op = CG.as_triton_op("logsumexp", lib="cpu_registry_test", keepdim=True, block=8192, num_warps=8)
    assert op is CG.as_triton_op("logsumexp", lib="cpu_registry_test", keepdim=True, block=8192, num_warps=8)
    handle = CG.op_handle("logsumexp", lib="cpu_registry_test", keepdim=True, block=8192, num_warps=8)
    assert isinstance(handle, torch._ops.OpOverload)
    assert str(handle).startswith("cpu_registry_test.logsumexp_keep_tiny0_b8192w8")
    with FakeTensorMode():
        assert handle(torch.empty(3, 5, 7)).shape == (3, 5, 1)
    seg = CG.segment_op_handle("segment_mean", {"initial": -2.0}, lib="cpu_registry_test")
    with FakeTensorMode():
        assert seg(torch.empty(3, 4), torch.empty(2, dtype=torch.int64)).shape == (2, 4)
    rms = CG.state_op_handle("rms_norm", {"eps": 1e-6}, lib="cpu_registry_test")
    with FakeTensorMode():
        assert rms(torch.empty(3, 8), torch.empty(8)).shape == (3, 8)
    attn = CG.as_attention_op(causal=True, lib="cpu_registry_test")
    with FakeTensorMode():
        q = torch.empty(1, 2, 5, 64, dtype=torch.bfloat16)
        assert attn(q, q, q).shape == q.shape


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(hip, "_lib", None)
    monkeypatch.setattr(hip, "LIB_PATH", tmp_path / "missing.so")
    with pytest.raises(RuntimeError, match="not built"):
        hip.load_library()


def test_attention_validation():
    q = meta((1, 2, 16, 128), torch.bfloat16)
    assert CG.run_attention(q, q, q).shape == q.shape
    with pytest.raises(TypeError, match="bfloat16"):
        CG.run_attention(meta((1, 2, 16, 128)), meta((1, 2, 16, 128)), meta((1, 2, 16, 128)))
    with pytest.raises(NotImplementedError, match="head_dim"):
        x = meta((1, 2, 16, 96), torch.bfloat16)
        CG.run_attention(x, x, x)
    with pytest.raises(ValueError, match="shapes"):
        CG.run_attention(q, meta((1, 2, 16, 64), torch.bfloat16), meta((1, 2, 16, 64), torch.bfloat16))
    with pytest.raises(ValueError, match="device"):
        x = torch.empty(1, 1, 4, 64, dtype=torch.bfloat16)
        CG.run_attention(x, x, x)
    for d, dt in ((256, torch.bfloat16), (64, torch.float16), (256, torch.float16)):
        x = meta((1, 2, 16, d), dt)
        out = CG.run_attention(x, x, x)
        assert out.shape == x.shape and out.dtype == dt
    with pytest.raises(TypeError, match="one dtype"):
        CG.run_attention(q, meta((1, 2, 16, 128), torch.float16), q)
