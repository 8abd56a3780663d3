"""Differential verification of a rewritten program against the original module.

`first_difference` walks two output pytrees and names the first disagreement: structure,
metadata, nonfinite classes (NaN, +inf and -inf positions must be identical), then values
within (rtol, atol), or -- for fp16/bf16 only, when the caller allows it -- within a number of
representable values (ULPs).  The difference texts are the reference's
(neptune_opt/__init__.py:76-114), which reports and callers match on.

`StateGuard` protects tensors a run must not change (parameters, buffers, an exported
program's state): it remembers each tensor's version counter and a copy, tells whether either
moved, and puts the saved values back.  `differential_run` executes module and candidate on
private copies of one argument tuple under such a guard and compares the results.
"""
from __future__ import annotations

import contextlib
import dataclasses

from neptune_opt.ab import _raise_if_fatal_cuda, fatal_cause


@dataclasses.dataclass(frozen=True)
class Tolerance:
    rtol: float = 1e-3
    atol: float = 1e-4
    max_ulps: int | None = None


EXACT = Tolerance(0.0, 0.0, None)


def ulp_distance(x, y):
    """Elementwise count of fp16/bf16 values between x and y.  Bit patterns become signed
    ordinals (sign-magnitude to two's complement), so +0 and -0 coincide and stepping across
    zero counts each value once."""
    import torch

    def ordinal(t):
        bits = t.contiguous().view(torch.int16).to(torch.int32)
        magnitude = bits & 0x7FFF
        return torch.where(bits < 0, -magnitude, magnitude)

    return (ordinal(x) - ordinal(y)).abs()


def _nonfinite_difference(index, x, y):
    import torch

    probes = [("finite classification", torch.isfinite), ("NaN classification", torch.isnan)]
    for what, probe in probes:
        if not torch.equal(probe(x), probe(y)):
            return f"output {index} {what} differs"
    if not x.is_complex():
        for probe in (torch.isposinf, torch.isneginf):
            if not torch.equal(probe(x), probe(y)):
                return f"output {index} infinity sign differs"
    return None


def _value_difference(index, x, y, tol: Tolerance):
    import torch

    try:
        torch.testing.assert_close(x, y, rtol=tol.rtol, atol=tol.atol, equal_nan=True)
        return None
    except AssertionError as error:
        _raise_if_fatal_cuda(error)
        if tol.max_ulps is None or x.dtype not in (torch.float16, torch.bfloat16):
            return f"output {index}: {error}"
    both_finite = torch.isfinite(x) & torch.isfinite(y)
    if bool((ulp_distance(x, y)[both_finite] <= tol.max_ulps).all()):
        return None
    return f"output {index}: exceeds explicit {tol.max_ulps}-ULP bound"


def _leaf_difference(index, x, y, tol: Tolerance):
    import torch

    if not (isinstance(x, torch.Tensor) and isinstance(y, torch.Tensor)):
        same = type(x) is type(y) and x == y
        return None if same else f"non-tensor output {index} differs"
    if (x.shape, x.dtype, x.device) != (y.shape, y.dtype, y.device):
        return f"output {index} shape/dtype/device differs"
    if not (x.is_floating_point() or x.is_complex()):
        return None if torch.equal(x, y) else f"output {index} integer/bool values differ"
    return _nonfinite_difference(index, x, y) or _value_difference(index, x, y, tol)


def first_difference(a, b, tol: Tolerance = Tolerance()):
    """None when the pytrees a and b agree under tol, else the first difference's text."""
    from torch.utils._pytree import tree_flatten

    left, left_spec = tree_flatten(a)
    right, right_spec = tree_flatten(b)
    if left_spec != right_spec:
        return "output pytree structure differs"
    for index, (x, y) in enumerate(zip(left, right)):
        difference = _leaf_difference(index, x, y, tol)
        if difference:
            return difference
    return None


def _compare_trees(a, b, *, rtol=1e-3, atol=1e-4, max_ulps=None):
    """(agree, difference text) -- the reference's comparison helper signature."""
    difference = first_difference(a, b, Tolerance(rtol, atol, max_ulps))
    return difference is None, difference or ""


def _version(tensor):
    try:
        return tensor._version
    except RuntimeError:            # inference tensors have no version counter
        return None


class StateGuard:
    """Remembers tensors (each distinct tensor once) so a run can be checked and undone."""

    def __init__(self, tensors):
        import torch

        distinct = {id(t): t for t in tensors if isinstance(t, torch.Tensor)}
        self._saved = [(t, _version(t), t.detach().clone()) for t in distinct.values()]

    def _moved(self, tensor, version, copy) -> bool:
        return _version(tensor) != version or first_difference(tensor, copy, EXACT) is not None

    def changed(self) -> bool:
        return any(self._moved(*entry) for entry in self._saved)

    def restore(self) -> None:
        import torch

        with torch.no_grad():
            for tensor, version, copy in self._saved:
                if self._moved(tensor, version, copy):
                    tensor.copy_(copy)


@contextlib.contextmanager
def guarded(tensors):
    """A StateGuard over `tensors` for the body of a with-statement.  On exit, normal or by
    an ordinary exception, the tensors get their saved values back; after a device-context
    failure nothing more may touch the GPU, so they are left as they are."""
    try:
        guard = StateGuard(tensors)
    except Exception as error:  # noqa: BLE001
        _raise_if_fatal_cuda(error)
        raise
    try:
        yield guard
    except BaseException as error:
        if fatal_cause(error) is None:
            _restore(guard)
        raise
    _restore(guard)


def _restore(guard):
    try:
        guard.restore()
    except Exception as error:  # noqa: BLE001
        _raise_if_fatal_cuda(error)
        raise


def _clones(args):
    import torch
    from torch.utils._pytree import tree_map

    return tree_map(lambda v: v.clone(memory_format=torch.preserve_format)
                    if isinstance(v, torch.Tensor) else v, args)


def _module_state(*modules):
    return [t for m in modules for t in (*m.parameters(), *m.buffers())]


def differential_run(module, candidate, args, tol: Tolerance = Tolerance()):
    """None when candidate reproduces module's outputs on args, else the reason.  Both run on
    private copies of args under no_grad; neither may change its parameters or buffers, nor
    its inputs.  Ordinary execution errors are reasons; a device-context failure raises."""
    with guarded(_module_state(module, candidate)) as guard:
        try:
            return _run_both(module, candidate, args, tol, guard)
        except Exception as error:  # noqa: BLE001 -- an ordinary execution error is a refusal
            _raise_if_fatal_cuda(error)
            return f"{type(error).__name__}: {error}"


def _run_both(module, candidate, args, tol, guard):
    import torch

    with torch.no_grad():
        mine, theirs = _clones(args), _clones(args)
        pristine = (_clones(mine), _clones(theirs))
        expected = module(*mine)
        if guard.changed():
            return "reference mutated parameters or buffers"
        got = candidate(*theirs)
        if guard.changed():
            return "candidate mutated parameters or buffers"
    for before, after in zip(pristine, (mine, theirs)):
        moved = first_difference(before, after, EXACT)
        if moved:
            return f"inputs mutated: {moved}"
    return first_difference(expected, got, tol)
