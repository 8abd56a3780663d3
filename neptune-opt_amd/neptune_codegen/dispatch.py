"""C++ dispatcher kernels for the row-fold operators: launch-plan replay.

An operator registered with torch.library.custom_op runs its Python body on every call (the
reference's Triton ops do the same, neptune_codegen/torch_op.py:16-114).  For the row folds
and the structured RMS / L2 operators that body is a pure function of the inputs' dtype,
device, sizes, strides and 16-byte alignment: it validates, picks a launch configuration,
allocates the output (and split scratch) and launches generated kernels through
`hip.Kernel.launch`, never reading tensor values on the host.  `install` gives such an
operator two C++ kernels (`_neptune_dispatch`, built from csrc/nep_dispatch.cpp):

  CUDA          first call per key: the Python body runs under `hip.recording`, and
                `plan_of` turns what it launched into a plan (buffer shapes, and per launch
                the packed kernarg image with the offsets of its pointer arguments, each tied
                to an input or a buffer).  Later calls with the same key allocate the buffers
                and replay the launches on the current stream without entering Python.
  AutogradCUDA  no input requires grad (or grad mode is off): straight to the CUDA kernel;
                otherwise the operator's original autograd kernel runs, as before.

A call whose body launches with a pointer that is neither an input nor a recorded buffer
(an input copied by reshape/contiguous, say) leaves no plan, and its key keeps using Python.
Bodies installed here must launch only through `hip.Kernel` and allocate scratch through
`hip.scratch`; the segment operators (device-side prefix sums and asserts) are not installed.
Plans are per process, at most MAX_PLANS (1024) per operator -- later layouts keep using the
Python body -- and hold only metadata; `clear()` drops them (after replacing the launch table,
for example).
"""
from __future__ import annotations

import importlib.util
import struct
import threading

from neptune_codegen import hip

_lock = threading.Lock()
_module = None
MAX_PLANS = 1024      # per operator; later layouts keep using the Python body
# qualname -> {"arguments": schema text after the name, "n_inputs": int,
#              "plans": {key tuple: (plan, kernels)}}: what export_bundle writes
_RECORDED: dict = {}
MODULE_PATH = hip.LIB_PATH.parent / "_neptune_dispatch.so"


def extension():
    """The loaded `_neptune_dispatch` module (raises when it has not been built)."""
    global _module
    with _lock:
        if _module is not None:
            return _module
        import torch  # noqa: F401  -- its libraries resolve the module's dependencies

        hip.load_library()
        if not MODULE_PATH.exists():
            raise RuntimeError(
                f"neptune dispatcher module is not built ({MODULE_PATH}); run "
                "`python -c 'import __graft_entry__ as g; g.build()'` from the repository root")
        spec = importlib.util.spec_from_file_location("_neptune_dispatch", MODULE_PATH)
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
        _module = module
        return module


def plan_of(recorder: hip.Recorder, inputs: tuple, outputs: tuple):
    """The replayable plan of one recorded call, or None when its launches use a pointer the
    plan cannot re-derive from the inputs and fresh buffers."""
    import torch

    if not all(isinstance(t, torch.Tensor) for t in outputs):
        return None
    buffers = list(outputs) + list(recorder.buffers)
    where: dict[int, int] = {}
    for i, t in enumerate(inputs):
        p = t.data_ptr()
        if p == 0 or p in where:
            return None
        where[p] = i
    for k, b in enumerate(buffers):
        p = b.data_ptr()
        if p == 0:
            if recorder.launches:
                return None
            continue
        if p in where:
            return None
        where[p] = -1 - k
    launches = []
    for kernel, grid, image, args in recorder.launches:
        patches = []
        for index, offset in kernel.pointer_offsets.items():
            value = int(args[index] or 0)
            if value == 0:
                continue
            source = where.get(value)
            if source is None:
                return None
            patches.append((offset, source))
        launches.append((kernel.handle, grid, kernel.block, kernel.lds, image, tuple(patches)))
    # buffers by metadata only: a plan must not keep the first call's tensors alive
    code = extension().dtype_code
    return (tuple((code(b), tuple(b.shape), tuple(b.stride())) for b in buffers),
            tuple(launches))


def install(qualname: str, n_inputs: int, body, *, backend: str = "CUDA") -> None:
    """Give the custom op `qualname` (already defined, tensor-only schema with one tensor
    output) its C++ CUDA and AutogradCUDA kernels; `body` is its Python implementation.
    backend="CPU" installs the same kernels on the CPU keys, for tests without a GPU."""
    import torch

    ext = extension()
    if ext.installed(qualname):
        return
    autograd_key = "Autograd" + backend
    original_autograd = torch._C._dispatch_get_computed_kernel_for_dispatch_key(
        qualname, autograd_key)
    # the keyset the dispatcher hands an autograd kernel: fallthrough keys already removed
    grad_keys = torch._C.DispatchKeySet(getattr(torch._C.DispatchKey, backend)).add(
        getattr(torch._C.DispatchKey, autograd_key))

    schema = str(torch._C._get_schema(qualname, ""))
    entry = {"arguments": schema[len(qualname):], "n_inputs": n_inputs, "plans": {}}

    def replayable_body(record, *inputs):
        if not record:
            return body(*inputs), None
        with hip.recording() as recorder:
            out = body(*inputs)
        plan = plan_of(recorder, inputs, (out,))
        if plan is not None:
            key = ext.key_of(list(inputs))
            if key is not None:
                with _lock:
                    if len(entry["plans"]) < MAX_PLANS:
                        entry["plans"][tuple(key)] = (plan, [k for k, *_ in recorder.launches])
        return out, plan

    def grad_body(*inputs):
        return original_autograd.call_boxed(grad_keys, *inputs)

    ext.install(qualname, n_inputs, replayable_body, grad_body, backend)
    with _lock:
        _RECORDED[qualname] = entry


def recorded_layouts(qualname: str) -> int:
    """How many input layouts of `qualname` have a recorded plan in this process."""
    with _lock:
        return len(_RECORDED.get(qualname, {}).get("plans", {}))


def export_bundle(path, qualnames=None) -> int:
    """Write the recorded launch plans of the installed operators (all, or `qualnames`) with
    their kernels' code objects to `path`, for libneptune_ops (`torch.ops.neptune_bundle.load`
    or `nep_ops_load_bundle`): a fused AOTI package then runs in a process without the Python
    package.  Only layouts this process ran are included.  Returns the number of plans."""
    ext = extension()
    with _lock:
        chosen = {q: e for q, e in _RECORDED.items()
                  if (qualnames is None or q in qualnames) and e["plans"]}
    if qualnames is not None:
        missing = set(qualnames) - set(chosen)
        if missing:
            raise ValueError(f"no recorded launch plan for {sorted(missing)}; run the operator "
                             "on the inputs to bundle first")
    codes: list[bytes] = []
    code_index: dict = {}
    ops_blob = bytearray()
    plans_written = 0

    def put_str(buf, text):
        data = text.encode()
        buf += struct.pack("<I", len(data)) + data

    ops_blob += struct.pack("<I", len(chosen))
    for qualname, entry in chosen.items():
        put_str(ops_blob, qualname)
        put_str(ops_blob, entry["arguments"])
        ops_blob += struct.pack("<II", entry["n_inputs"], len(entry["plans"]))
        for key, ((buffers, launches), kernels) in entry["plans"].items():
            ops_blob += struct.pack("<I", len(key)) + struct.pack(f"<{len(key)}q", *key)
            ops_blob += struct.pack("<I", len(buffers))
            for dtype_code, sizes, strides in buffers:
                ops_blob += struct.pack("<iI", dtype_code, len(sizes))
                ops_blob += struct.pack(f"<{len(sizes)}q", *sizes)
                ops_blob += struct.pack(f"<{len(strides)}q", *strides)
            ops_blob += struct.pack("<I", len(launches))
            for (_handle, grid, block, lds, image, patches), kernel in zip(launches, kernels):
                program = kernel.program
                ident = (program.source, program.options)
                if ident not in code_index:
                    code_index[ident] = len(codes)
                    codes.append(program.code_object())
                ops_blob += struct.pack("<I", code_index[ident])
                put_str(ops_blob, kernel.name)
                ops_blob += struct.pack("<5I", *grid, block, lds)
                ops_blob += struct.pack("<I", len(image)) + image
                ops_blob += struct.pack("<I", len(patches))
                for offset, source in patches:
                    ops_blob += struct.pack("<Ii", offset, source)
            plans_written += 1
    blob = bytearray(b"NEPBNDL1") + struct.pack("<I", len(codes))
    for code in codes:
        blob += struct.pack("<I", len(code)) + code
    blob += ops_blob
    with open(path, "wb") as f:
        f.write(bytes(blob))
    return plans_written


OPS_LIBRARY = hip.LIB_PATH.parent / "libneptune_ops.so"


def stats(qualname: str) -> dict:
    """{'replays', 'python_calls', 'plans'} of an installed operator."""
    return dict(extension().stats(qualname))


def clear() -> None:
    """Drop every recorded plan (the next call per key runs the Python body again)."""
    extension().clear()
