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
Plans are per process; `clear()` drops them (after replacing the launch table, for example).
"""
from __future__ import annotations

import importlib.util
import threading

from neptune_codegen import hip

_lock = threading.Lock()
_module = None
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
    return tuple((b,) for b in buffers), tuple(launches)


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

    def replayable_body(record, *inputs):
        if not record:
            return body(*inputs), None
        with hip.recording() as recorder:
            out = body(*inputs)
        return out, plan_of(recorder, inputs, (out,))

    def grad_body(*inputs):
        return original_autograd.call_boxed(grad_keys, *inputs)

    ext.install(qualname, n_inputs, replayable_body, grad_body, backend)


def stats(qualname: str) -> dict:
    """{'replays', 'python_calls', 'plans'} of an installed operator."""
    return dict(extension().stats(qualname))


def clear() -> None:
    """Drop every recorded plan (the next call per key runs the Python body again)."""
    extension().clear()
