"""Custom-op bridge and the segment-pooling backend.

Mirrors the reference's neptune_codegen/torch_op.py: op naming from `autotune.op_key`
(as_triton_op :16-114, op_handle :117-134), the structured two-input op (as_state_op
:145-190), and the whole segment backend -- parameter validation, span construction with
device-side asserts, metadata contract, launch and op registration (:208-466).  Ops are
registered with torch.library.custom_op (schema identical to the reference's triton_op) and
a metadata-only fake; their bodies launch generated HIP kernels through libneptune_hip.  The
row-fold and RMS / L2 operators also get C++ dispatcher kernels that replay a recorded launch
plan per input layout (neptune_codegen.dispatch).
"""
from __future__ import annotations

import threading

from neptune_codegen import autotune, dispatch, hip
from neptune_codegen.emitters import (BASE_OPTIONS, NO_CONTRACT, SegmentVariant,
                                      emit_segment_source, segment_kernel_name)
from neptune_codegen.skeleton import param_defaults
from neptune_codegen.template import (_row_last_layout, _validate_row_last, compile_skeleton,
                                      launch_reduction, split_launch_shape, validate_plan)

_TRITON_OPS: dict[str, object] = {}
_lock = threading.Lock()


def _register(qualname: str, schema: str, impl, fake):
    import torch

    op = torch.library.custom_op(qualname, mutates_args=(), schema=schema)(impl)
    op.register_fake(fake)
    return op


def as_triton_op(name: str, block: int | None = None, num_warps: int | None = None,
                 lib: str = "neptune", params: dict | None = None, keepdim: bool = False,
                 plan: str = "serial"):
    """Register the generated fold `name` as the custom op `lib::<op_key>` (schema
    `(Tensor x) -> Tensor`); the name encodes parameters, rank and a fixed launch config."""
    validate_plan(plan)
    if plan == "split":
        block = 1024 if block is None else block
        num_warps = 4 if num_warps is None else num_warps
    params = {**param_defaults(name), **(params or {})}
    key = autotune.op_key(lib, name, params, keepdim, block, num_warps)
    if plan != "serial":
        key += "_plan_split"
        from neptune_codegen.algebra import derive_merge_certificate
        from neptune_codegen.skeleton import SKELETONS

        derive_merge_certificate(SKELETONS[name], params)
    with _lock:
        if key in _TRITON_OPS:
            return _TRITON_OPS[key]
    import torch

    kernel = compile_skeleton(name, params, plan=plan)
    impl_name = key.split("::", 1)[1]

    def _impl(x):
        _validate_row_last(x)
        x2, rows, ncols = _row_last_layout(x)
        out = torch.empty(x.shape[:-1] + ((1,) if keepdim else ()), device=x.device, dtype=x.dtype)
        if isinstance(rows, int) and rows == 0:
            return out
        cfg = (block, num_warps)
        if block is None or num_warps is None:
            chosen = autotune.best_config(rows, ncols, x.dtype, x.device)
            cfg = (chosen[0] if block is None else block, chosen[1] if num_warps is None else num_warps)
        launch_reduction(kernel, plan, x2, out, rows, ncols, cfg[0], cfg[1])
        return out

    def _fake(x):
        _validate_row_last(x, metadata=True)
        if plan == "split":
            split_launch_shape(x.shape[-1], block if block is not None else 1024)
        return torch.empty(x.shape[:-1] + ((1,) if keepdim else ()), device=x.device, dtype=x.dtype)

    op = _register(key, "(Tensor x) -> Tensor", _impl, _fake)
    dispatch.install(key, 1, _impl)
    op.__name__ = f"{lib}_{impl_name}"
    with _lock:
        _TRITON_OPS[key] = op
    return op


# The op is a HIP kernel, not Triton; the reference's name stays for drop-in callers.
as_hip_op = as_triton_op


def _overload(lib: str, impl):
    import torch

    packet = getattr(getattr(torch.ops, lib), impl.__name__[len(lib) + 1:])
    return getattr(packet, "default", packet)


def op_handle(name: str, params: dict | None = None, lib: str = "neptune", keepdim: bool = False,
              block: int | None = None, num_warps: int | None = None, plan: str = "serial"):
    """The OpOverload of a compiled skeleton, for building graph nodes."""
    impl = as_triton_op(name, block=block, num_warps=num_warps, params=params, lib=lib,
                        keepdim=keepdim, plan=plan)
    return _overload(lib, impl)


def triton_op_name(name: str, lib: str = "neptune") -> str:
    return f"{lib}.{name}"


def as_readout_op(name: str, params: dict | None = None, nan_posinf_rows: bool = True,
                  lib: str = "neptune", block: int | None = None, num_warps: int | None = None):
    """Custom op `(Tensor x) -> Tensor`: the readout phi(x) - r of the exponential fold `name`
    (log_softmax for logsumexp), output of x's shape and dtype.  The name is the fold's op key
    plus `_readout` (`_readout_nanrows` when +inf rows read out NaN)."""
    from neptune_codegen.template import compile_readout, launch_readout

    params = {**param_defaults(name), **(params or {})}
    key = autotune.op_key(lib, name, params, False, block, num_warps)
    key += "_readout_nanrows" if nan_posinf_rows else "_readout"
    with _lock:
        if key in _TRITON_OPS:
            return _TRITON_OPS[key]
    import torch

    program = compile_readout(name, params, nan_posinf_rows=nan_posinf_rows)
    impl_name = key.split("::", 1)[1]

    def _impl(x):
        _validate_row_last(x)
        x2, rows, ncols = _row_last_layout(x)
        out = torch.empty(x.shape, device=x.device, dtype=x.dtype)
        if isinstance(rows, int) and rows == 0:
            return out
        cfg = (block, num_warps)
        if block is None or num_warps is None:
            chosen = autotune.best_config(rows, ncols, x.dtype, x.device)
            cfg = (chosen[0] if block is None else block, chosen[1] if num_warps is None else num_warps)
        launch_readout(program, x2, out, rows, ncols, cfg[0], cfg[1])
        return out

    def _fake(x):
        _validate_row_last(x, metadata=True)
        return torch.empty(x.shape, device=x.device, dtype=x.dtype)

    op = _register(key, "(Tensor x) -> Tensor", _impl, _fake)
    dispatch.install(key, 1, _impl)
    op.__name__ = f"{lib}_{impl_name}"
    with _lock:
        _TRITON_OPS[key] = op
    return op


def readout_op_handle(name: str, params: dict | None = None, nan_posinf_rows: bool = True,
                      lib: str = "neptune", block: int | None = None,
                      num_warps: int | None = None):
    """The OpOverload of a fold's readout op, for building graph nodes."""
    return _overload(lib, as_readout_op(name, params=params, nan_posinf_rows=nan_posinf_rows,
                                        lib=lib, block=block, num_warps=num_warps))


# ---------------------------------------------------------------- structured row ops
_STATE_OPS: dict[tuple, object] = {}


def as_state_op(name, params=None, plan="serial", lib="neptune"):
    """Structured op: rms_norm `(Tensor x, Tensor gamma) -> Tensor`, l2_normalize
    `(Tensor x) -> Tensor`; segment names go to as_segment_op."""
    import torch

    from neptune_codegen.algebra import derive_state_certificate
    from neptune_codegen.emitters import emit_rms_state_source
    from neptune_codegen.skeleton import state_reduction_spec
    from neptune_codegen.template import (compile_state_reduction, launch_rms_norm,
                                          validate_l2_inputs, validate_rms_inputs)

    spec = state_reduction_spec(name)
    derive_state_certificate(spec)
    if name in ("segment_sum", "segment_mean"):
        return as_segment_op(name, params=params, plan=plan, lib=lib)
    validate_plan(plan)
    params = dict(params or {})
    emit_rms_state_source(spec, params, plan=plan)
    key = (lib, spec, autotune.parameter_identity(params), plan)
    with _lock:
        if key in _STATE_OPS:
            return _STATE_OPS[key]
    impl_name = f"state_{name}{autotune.parameter_tag(params)}_plan_{plan}"
    if name == "rms_norm":
        def _impl(x, gamma):
            shape = validate_rms_inputs(x, gamma, params, plan=plan)
            out = torch.empty(shape, dtype=x.dtype, device=x.device)
            if x.numel() == 0:
                return out
            launch_rms_norm(compile_state_reduction(name, params, plan=plan), x, gamma, out, plan=plan)
            return out

        def _fake(x, gamma):
            shape = validate_rms_inputs(x, gamma, params, plan=plan, metadata=True)
            return torch.empty(shape, dtype=x.dtype, device=x.device)

        schema = "(Tensor x, Tensor gamma) -> Tensor"
    else:
        def _impl(x):
            shape = validate_l2_inputs(x, params, plan=plan)
            out = torch.empty(shape, dtype=x.dtype, device=x.device)
            if x.numel() == 0:
                return out
            launch_rms_norm(compile_state_reduction(name, params, plan=plan), x, None, out, plan=plan)
            return out

        def _fake(x):
            shape = validate_l2_inputs(x, params, plan=plan, metadata=True)
            return torch.empty(shape, dtype=x.dtype, device=x.device)

        schema = "(Tensor x) -> Tensor"
    op = _register(f"{lib}::{impl_name}", schema, _impl, _fake)
    dispatch.install(f"{lib}::{impl_name}", 2 if name == "rms_norm" else 1, _impl)
    op.__name__ = f"{lib}_{impl_name}"
    with _lock:
        _STATE_OPS[key] = op
    return op


def state_op_handle(name, params=None, plan="serial", lib="neptune"):
    return _overload(lib, as_state_op(name, params=params, plan=plan, lib=lib))


# ---------------------------------------------------------------- segment backend
_SEGMENT_KERNELS: dict[tuple, object] = {}
_SEGMENT_OPS: dict[tuple, object] = {}
_SEGMENT_NAMES: dict[str, tuple] = {}


def _segment_params(name, params=None, plan="serial"):
    """Validated (initial, offsets, unsafe) of a segment reduction (torch_op.py:208-232)."""
    import math

    if name not in ("segment_sum", "segment_mean"):
        raise KeyError(f"unknown segment reduction {name!r}")
    from neptune_codegen.skeleton import state_reduction_spec

    state_reduction_spec(name)
    validate_plan(plan)
    if plan != "serial":
        raise NotImplementedError("segment split cannot preserve ordered storage-dtype rounding; use serial")
    params = dict(params or {})
    unknown = params.keys() - {"initial", "offsets", "unsafe"}
    if unknown:
        raise ValueError(f"unknown segment parameters: {sorted(unknown)}")
    initial = params.get("initial")
    if initial is not None:
        if isinstance(initial, bool) or not isinstance(initial, (int, float)):
            raise TypeError("segment initial must be a finite Python scalar or None")
        initial = float(initial)
        if not math.isfinite(initial):
            raise ValueError("segment initial must be finite")
    offsets, unsafe = params.get("offsets", False), params.get("unsafe", False)
    if type(offsets) is not bool or type(unsafe) is not bool:
        raise TypeError("segment offsets and unsafe must be bool")
    return {"initial": initial, "offsets": offsets, "unsafe": unsafe}


def _segment_identity(name, params, plan):
    numeric = {k: v for k, v in params.items() if v is not None}
    # (64, 4) is the reference's launch tuple; kept so registered op names stay identical.
    return (name, params["initial"] is None, autotune.parameter_identity(numeric), plan, 64, 4)


def _segment_module_name(identity):
    import hashlib

    stem = f"neptune_gen_{identity[0]}_serial_h" + hashlib.sha256(repr(identity).encode()).hexdigest()[-10:]
    candidate, collision = stem, 0
    while candidate in _SEGMENT_NAMES and _SEGMENT_NAMES[candidate] != identity:
        collision += 1
        candidate = f"{stem}_{collision}"
    _SEGMENT_NAMES[candidate] = identity
    return candidate


class SegmentProgram:
    """Generated segment kernels of one identity; launch variants compile lazily."""

    def __init__(self, name: str, params: dict, plan: str):
        self.name, self.params, self.plan = name, dict(params), plan
        self._programs: dict = {}

    def source(self, var: SegmentVariant) -> str:
        return emit_segment_source(self.name, initial=self.params["initial"],
                                   offsets=self.params["offsets"], plan=self.plan, variants=(var,))

    def program(self, var: SegmentVariant) -> hip.Program:
        prog = self._programs.get(var)
        if prog is None:
            prog = hip.Program(self.source(var), f"{self.name}_{var.tag()}.hip",
                               BASE_OPTIONS + NO_CONTRACT)
            self._programs[var] = prog
        return prog

    def kernel(self, var: SegmentVariant, device: int) -> hip.Kernel:
        return self.program(var).kernel(segment_kernel_name(self.name, var),
                                        (hip.PTR,) * 3 + (hip.I64,) * 6 + (hip.PTR, hip.I64),
                                        256 if var.vector else 64, device)


def compile_segment_reduction(name, params=None, plan="serial"):
    """The cached SegmentProgram for an exact parameter identity."""
    params = _segment_params(name, params, plan)
    identity = _segment_identity(name, params, plan)
    with _lock:
        if identity in _SEGMENT_KERNELS:
            return _SEGMENT_KERNELS[identity]
    emit_segment_source(name, initial=params["initial"], offsets=params["offsets"], plan=plan)
    program = SegmentProgram(name, params, plan)
    with _lock:
        _segment_module_name(identity)
        _SEGMENT_KERNELS[identity] = program
    return program


def validate_segment_inputs(data, segments, *, metadata=False, offsets=False,
                            initial=None, unsafe=False, reduce="sum", plan="serial"):
    """Metadata-only contract (torch_op.py:340-367); returns the output shape."""
    import torch

    _segment_params("segment_" + reduce, {"initial": initial, "offsets": offsets, "unsafe": unsafe}, plan)
    if data.layout != torch.strided or segments.layout != torch.strided:
        raise TypeError("segment requires strided data and segments")
    if data.ndim < 1 or segments.ndim != 1:
        raise ValueError("segment data rank must be >= 1 and segments rank must be 1")
    if data.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError("segment data dtype must be float16/bfloat16/float32")
    if initial is not None and abs(initial) > torch.finfo(data.dtype).max:
        raise RuntimeError("segment initial cannot be converted to input dtype without overflow")
    if segments.dtype not in (torch.int32, torch.int64):
        raise TypeError("segment index dtype must be int32/int64")
    if data.device != segments.device:
        raise ValueError("segment tensors must be on the same device")
    if not metadata and data.device.type != "cuda":
        raise ValueError("segment execution requires a CUDA (ROCm) device")
    if offsets:
        torch._check(segments.shape[0] >= 1, lambda: "segment offsets needs at least one boundary")
    count = segments.shape[0] - 1 if offsets else segments.shape[0]
    return (count,) + data.shape[1:]


def _segment_spans(data, segments, *, offsets, unsafe):
    """[start, end) boundaries; lengths become int64 prefix sums; device-side asserts check
    range, coverage (unless unsafe) and monotonicity (torch_op.py:370-387)."""
    import torch

    nrows = data.shape[0]
    if offsets:
        spans = segments
    else:
        torch._assert_async(torch.all((segments >= 0) & (segments <= nrows)),
                            "segment lengths must be nonnegative and within data bounds")
        spans = torch.cat((segments.new_zeros((1,), dtype=torch.int64),
                           torch.cumsum(segments, dim=0, dtype=torch.int64)))
        if not unsafe:
            torch._assert_async(spans[-1] == nrows, "segment lengths must sum to data axis0 size")
    torch._assert_async(torch.all((spans >= 0) & (spans <= nrows)), "segment boundaries out of data bounds")
    torch._assert_async(torch.all(spans[1:] >= spans[:-1]), "segment boundaries must be monotonic")
    return spans


def _segment_variant(flat, spans, channels: int) -> SegmentVariant:
    from neptune_codegen.autotune import vec_of

    dtype = str(flat.dtype).replace("torch.", "")
    span_dtype = str(spans.dtype).replace("torch.", "")
    vec = vec_of(flat.dtype)
    lanes = channels // vec if channels % vec == 0 else 0
    vector = (lanes > 0 and lanes <= 64 and lanes & (lanes - 1) == 0
              and (flat.stride(1) == 1 or channels == 1) and flat.stride(0) % vec == 0
              and flat.data_ptr() % 16 == 0)
    if vector:
        # 16 tokens in flight per lane: cfg4 (Poisson(20) segments, 128 fp16 channels) 55.8 us
        # against 58.6 us at 8 tokens and 57.3 us at 32, bit-identical results
        return SegmentVariant(dtype, span_dtype, True, lanes, 16)
    return SegmentVariant(dtype, span_dtype, False, 64, 4)


DESCRIPTOR_MESSAGE = ("segment descriptor is invalid: lengths must be nonnegative, within data bounds "
                      "and (unless unsafe) sum to data axis0 size; boundaries must lie within data "
                      "bounds and be monotonic")


_SPANS_PROGRAM = None


def _spans_program() -> hip.Program:
    global _SPANS_PROGRAM
    with _lock:
        if _SPANS_PROGRAM is None:
            from neptune_codegen.emitters import emit_segment_spans_source

            _SPANS_PROGRAM = hip.Program(emit_segment_spans_source(), "segment_spans.hip",
                                         BASE_OPTIONS)
        return _SPANS_PROGRAM


def _device_spans(data, segments, *, offsets, status=None):
    """[start, end) boundaries for the fused-validation launch: offsets as given, lengths as an
    int64 prefix sum (the same values `_segment_spans` builds) by two HIP launches -- block
    sums, then a per-block scan on top of the preceding blocks; no asserts here (the segment
    kernel checks the spans).  With lengths, the first launch also sets `status` (one int32)
    to 1; returns (spans, status set)."""
    import torch

    from neptune_codegen.emitters import SPAN_BLOCK

    if offsets:
        return segments, False
    lengths = segments.contiguous()
    n = lengths.shape[0]
    spans = torch.empty(n + 1, dtype=torch.int64, device=segments.device)
    nblocks = (n + SPAN_BLOCK - 1) // SPAN_BLOCK
    sums = hip.scratch(torch.empty(nblocks, dtype=torch.int64, device=segments.device))
    tag = "i32" if lengths.dtype == torch.int32 else "i64"
    device = segments.device.index if segments.device.index is not None else torch.cuda.current_device()
    prog = _spans_program()
    stream = hip.current_stream(segments.device)
    prog.kernel(f"segment_spans_sums_{tag}", (hip.PTR, hip.I64, hip.PTR, hip.PTR), 256,
                device).launch((nblocks,), (lengths.data_ptr(), n, sums.data_ptr(),
                                            status.data_ptr() if status is not None else 0),
                               stream)
    prog.kernel(f"segment_spans_scan_{tag}", (hip.PTR, hip.I64, hip.PTR, hip.PTR), 256,
                device).launch((nblocks,), (lengths.data_ptr(), n, sums.data_ptr(),
                                            spans.data_ptr()), stream)
    return spans, status is not None


def _launch_segment(name, data, segments, params, plan, *, wrapper=None):
    """The segment op body.  With at least one segment and channel, the reference's span
    asserts (range, coverage unless unsafe, monotonic) are evaluated inside the fold kernel,
    which clears the device's one-word status (armed once); one `_assert_async` on it follows,
    on the same stream.
    Otherwise the spans are built and asserted exactly as `_segment_spans` does."""
    import torch

    # CSR offsets seen before with the same tensor layout and parameters: the validation, the
    # variant and the launch shape are what that call found; only the output allocation, the
    # launch (span checks inside) and the assert on the armed status word remain
    key = None
    if (params["offsets"] and type(data) is torch.Tensor and type(segments) is torch.Tensor
            and data.is_cuda and not hip.recording_active()):
        try:
            key = (name, plan, tuple(sorted((k, type(v).__name__, repr(v)) for k, v in params.items())),
                   data.dtype, data.device, tuple(data.shape), tuple(data.stride()),
                   data.data_ptr() % 16, segments.dtype, segments.device, tuple(segments.shape),
                   tuple(segments.stride()))
            entry = _SEG_SEEN.get(key)
        except TypeError:
            key, entry = None, None
        status = _armed_status(data.device) if entry is not None else None
        if status is not None:
            out_shape, kernel, grid, tail = entry
            out = torch.empty(out_shape, dtype=data.dtype, device=data.device)
            kernel.launch(grid, (data.data_ptr(), segments.data_ptr(), out.data_ptr()) + tail,
                          hip.current_stream(data.device))
            torch._assert_async(status, DESCRIPTOR_MESSAGE)
            return out
    shape = validate_segment_inputs(data, segments, reduce=name.removeprefix("segment_"),
                                    plan=plan, **params)
    channels = 1
    for size in data.shape[1:]:
        channels = channels * size
    out = torch.empty(shape, dtype=data.dtype, device=data.device)
    nseg = shape[0]
    if type(nseg) is int and nseg > 0 and type(channels) is int and channels > 0:
        status = _armed_status(data.device)
        if status is None:      # first call on this device under graph capture
            status = torch.empty(1, dtype=torch.int32, device=data.device)
            spans, status_set = _device_spans(data, segments, offsets=params["offsets"],
                                              status=status)
            if not status_set:
                status.fill_(1)
        else:
            spans, _ = _device_spans(data, segments, offsets=params["offsets"])
        cover = -1 if params["offsets"] or params["unsafe"] else data.shape[0]
        flat = data.reshape(data.shape[0], channels)
        launch = launch_segment_kernel(compile_segment_reduction(name, params, plan), flat, spans,
                                       out, status=status, cover=cover)
        torch._assert_async(status, DESCRIPTOR_MESSAGE)
        if (key is not None and flat.data_ptr() == data.data_ptr() and spans is segments
                and status is _STATUS.get(data.device.index if data.device.index is not None
                                          else torch.cuda.current_device())):
            if len(_SEG_SEEN) >= 4096:
                _SEG_SEEN.clear()
            _SEG_SEEN[key] = (tuple(out.shape),) + launch
        return out
    _segment_spans(data, segments, offsets=params["offsets"], unsafe=params["unsafe"])
    return out


_STATUS: dict = {}
_SEG_SEEN: dict = {}


def _armed_status(device):
    """The device's span-check status word: one int32 set to 1 once, outside graph capture.
    A kernel clears it only for a malformed descriptor, and the `_assert_async` on it then
    ends the device context, so no call needs to re-arm it.  None while capturing before the
    word exists (the caller then arms a fresh word in the captured stream)."""
    import torch

    index = device.index if device.index is not None else torch.cuda.current_device()
    word = _STATUS.get(index)
    if word is None:
        if torch.cuda.is_current_stream_capturing():
            return None
        with _lock:
            word = _STATUS.get(index)
            if word is None:
                word = torch.ones(1, dtype=torch.int32, device=torch.device("cuda", index))
                _STATUS[index] = word
    return word


def launch_segment_kernel(program, flat, spans, out, *, status=None, cover=-1):
    """The fold launch alone: flat [nrows, channels] data, spans [nsegments + 1], out
    [nsegments, channels] (contiguous).  `status` (one int32 set to 1, or None) receives 0 when
    a span is malformed or, with cover >= 0, the last span does not end at `cover`."""
    import torch

    channels = flat.shape[1]
    nseg = spans.shape[0] - 1
    var = _segment_variant(flat, spans, channels)
    device = flat.device.index if flat.device.index is not None else torch.cuda.current_device()
    kernel = program.kernel(var, device)
    if var.vector:
        grid = (max(1, -(-nseg // (256 // var.lps))),)
    else:
        grid = (nseg, -(-channels // 64))
    tail = (flat.shape[0], channels, nseg, flat.stride(0), flat.stride(1), spans.stride(0),
            status.data_ptr() if status is not None else 0, int(cover))
    kernel.launch(grid, (flat.data_ptr(), spans.data_ptr(), out.data_ptr()) + tail,
                  hip.current_stream(flat.device))
    return kernel, grid, tail


def run_segment_pool(data, segments, *, reduce="sum", offsets=False, initial=None,
                     unsafe=False, plan="serial"):
    """Direct segment sum/mean; Fake/meta calls return metadata only."""
    import torch
    from torch._subclasses.fake_tensor import FakeTensor

    name = "segment_" + reduce
    params = _segment_params(name, {"initial": initial, "offsets": offsets, "unsafe": unsafe}, plan)
    if data.device.type == "meta" or isinstance(data, FakeTensor):
        shape = validate_segment_inputs(data, segments, metadata=True, reduce=reduce, plan=plan, **params)
        return torch.empty(shape, dtype=data.dtype, device=data.device)
    return _launch_segment(name, data, segments, params, plan)


def as_segment_op(name, params=None, plan="serial", lib="neptune"):
    """Custom op `(Tensor data, Tensor segments) -> Tensor`; constants live in its identity."""
    import torch

    params = _segment_params(name, params, plan)
    identity = (lib, _segment_identity(name, params, plan))
    with _lock:
        if identity in _SEGMENT_OPS:
            return _SEGMENT_OPS[identity]
        impl_name = _segment_module_name(identity[1]).removeprefix("neptune_gen_")

    def _impl(data, segments):
        return _launch_segment(name, data, segments, params, plan)

    def _fake(data, segments):
        shape = validate_segment_inputs(data, segments, metadata=True,
                                        reduce=name.removeprefix("segment_"), plan=plan, **params)
        return torch.empty(shape, dtype=data.dtype, device=data.device)

    op = _register(f"{lib}::{impl_name}", "(Tensor data, Tensor segments) -> Tensor", _impl, _fake)
    op.__name__ = f"{lib}_{impl_name}"
    with _lock:
        _SEGMENT_OPS[identity] = op
    return op


def segment_op_handle(name, params=None, plan="serial", lib="neptune"):
    return _overload(lib, as_segment_op(name, params=params, plan=plan, lib=lib))
