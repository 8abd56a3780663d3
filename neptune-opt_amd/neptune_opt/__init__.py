"""neptune_opt -- transactional reduction fusion into MI355X HIP folds.

The public API of the reference package (neptune_opt/__init__.py:26-604): `apply` rewrites
recognised regions of an ExportedProgram into fused HIP ops, verifies them against the
original module on supplied inputs, and publishes the new graph only when every step
succeeded; `preview` reports what `apply` would do; `export` is export + apply; one function
per supported skeleton calls the fused op directly; `compile_best` measures AOTI packages.
Real-algebra matching is a legality check, not an IEEE proof; verification covers the
supplied cases.  A failed trial never changes the caller's graph, signature or weights.

The work is split by concern: report.py (Fusion, Report), transaction.py (trial graphs, the
region pass, the signature rebuild), verification.py (differential runs and output
comparison), ab.py (compile_best).
"""
from __future__ import annotations

import math
import sys
import warnings
from collections.abc import Iterable, Sequence

import torch

import neptune_codegen as CG
from neptune_opt import transaction as _tx
from neptune_opt.ab import (Choice, FatalCudaError, _bounded_names, _raise_if_fatal_cuda,
                            choose_faster, compile_best)
from neptune_opt.report import Fusion, Report
from neptune_opt.verification import Tolerance, _compare_trees, differential_run, guarded
from neptune_recognize.rewrite import region_contract

__all__ = ["apply", "export", "optimize", "backend", "preview", "Report", "Fusion",
           "LAST_REPORT", "op_parameters", "compile_best", "Choice"]

LAST_REPORT: Report | None = None

# the reference's refusal texts for a bad `capabilities` argument of apply/preview
_CAPABILITY_MESSAGES = {
    "not_iterable": "capabilities must be an iterable of capability names",
    "string": "capabilities must be an iterable of distinct capability names",
    "bad_item": "capabilities must contain only distinct rms_norm/segment_pool names",
    "too_many": "at most two capabilities are supported",
}


def _capabilities(capabilities: Iterable[str]) -> tuple:
    return _bounded_names(capabilities, ("rms_norm", "segment_pool"), _CAPABILITY_MESSAGES)


def _is_count(value, least) -> bool:
    return type(value) is int and value >= least


# apply's argument checks, in order: (is the argument acceptable, ValueError text)
_ARGUMENT_CHECKS = (
    (lambda o: o["max_regions"] is None or _is_count(o["max_regions"], 1),
     "max_regions must be a positive integer or None"),
    (lambda o: all(math.isfinite(t) and t >= 0 for t in (o["rtol"], o["atol"])),
     "verification tolerances must be finite and nonnegative"),
    (lambda o: o["max_ulps"] is None or _is_count(o["max_ulps"], 0),
     "max_ulps must be a nonnegative integer or None"),
    (lambda o: o["cases"] is None or isinstance(o["cases"], Sequence),
     "verification_inputs must be a sequence of argument tuples"),
    (lambda o: o["cases"] is None or all(isinstance(c, tuple) for c in o["cases"]),
     "each verification_inputs sample must be an argument tuple"),
)


def _checked_options(plan, capabilities, max_regions, rtol, atol, max_ulps, verification_inputs):
    """(capabilities, Tolerance); ValueError names the first bad argument."""
    from neptune_codegen.template import validate_plan

    validate_plan(plan)
    capabilities = _capabilities(capabilities)
    given = {"max_regions": max_regions, "rtol": rtol, "atol": atol, "max_ulps": max_ulps,
             "cases": verification_inputs}
    for acceptable, message in _ARGUMENT_CHECKS:
        if not acceptable(given):
            raise ValueError(message)
    return capabilities, Tolerance(rtol, atol, max_ulps)


def _first_failing_case(exported, candidate, verify_with, verification_inputs, tol):
    """None when the candidate reproduces the module on every case, else (case index, reason).
    The exported program's own state is guarded too: a reference module may hold it through
    a closure rather than as a submodule."""
    module, args = verify_with
    cases = [tuple(args), *(tuple(case) for case in verification_inputs or ())]
    executable = candidate.module()
    state = [*exported.state_dict.values(), *exported.constants.values()]
    for index, case in enumerate(cases):
        with guarded(state) as guard:
            reason = differential_run(module, executable, case, tol)
            if guard.changed():
                reason = "verification mutated original exported state"
        if reason is not None:
            return index, reason
    return None


def _transaction(exported, values, verify_with, lower, experimental_log_softmax, plan,
                 max_regions, verification_inputs, capabilities, tol) -> Report:
    signature = exported.graph_signature
    if signature.buffers_to_mutate or signature.user_inputs_to_mutate:
        raise ValueError("state/input mutation is outside inference reduction fusion")
    trial = _tx.fork(exported.graph_module)
    report = _tx.fuse_regions(trial, values, plan=plan, max_regions=max_regions, lower=lower,
                              experimental_log_softmax=experimental_log_softmax,
                              capabilities=capabilities)
    if not report.fusions:
        return report
    candidate = _tx.program_with(exported, trial)
    if verify_with is not None:
        failure = _first_failing_case(exported, candidate, verify_with, verification_inputs, tol)
        if failure is not None:
            index, reason = failure
            return Report(skipped=[("verify-failed", f"case {index}: {reason}")],
                          verification_cases=index + 1)
        report.verified = True
        report.verification_cases = 1 + len(verification_inputs or ())
    _tx.publish(exported, candidate)
    report.graph_changed = True
    return report


def apply(exported_program, values: dict | None = None, verify_with: tuple | None = None,
          lower: bool = True, *, plan="serial", max_regions=None,
          verification_inputs=None, rtol=1e-3, atol=1e-4,
          experimental_log_softmax=False, max_ulps=None,
          capabilities: Iterable[str] = ()) -> Report:
    """Fuse recognised regions of `exported_program` in place, transactionally.

    Unknown ops, casts and other inputs remain boundaries.  Compound lowering covers LSE (and,
    with experimental_log_softmax, the x - LSE readout).  With `verify_with=(module, args)` the
    candidate must reproduce module's outputs on args and every `verification_inputs` case;
    without it the report says UNVERIFIED.  Any failure leaves the program unchanged and is
    reported in the returned Report (also stored in LAST_REPORT); a fatal HIP context error
    propagates as FatalCudaError."""
    global LAST_REPORT
    try:
        capabilities, tol = _checked_options(plan, capabilities, max_regions, rtol, atol,
                                             max_ulps, verification_inputs)
        report = _transaction(exported_program, values, verify_with, lower,
                              experimental_log_softmax, plan, max_regions, verification_inputs,
                              capabilities, tol)
    except Exception as error:  # noqa: BLE001 -- an optional optimisation fails closed
        _raise_if_fatal_cuda(error)
        report = Report(skipped=[("rewrite-failed", f"{type(error).__name__}: {error}")])
    LAST_REPORT = report
    return report


def preview(exported_program, values: dict | None = None, *, lower=True,
            experimental_log_softmax=False, capabilities: Iterable[str] = ()):
    """(eligible matches, reason) that apply would rewrite; generates and launches nothing."""
    capabilities = _capabilities(capabilities)
    trial = _tx.fork(exported_program.graph_module)
    if lower:
        for _, lowered, _ in _tx.lowered_regions(trial, values, experimental_log_softmax):
            _tx.install(trial, lowered)
    matches, reason = _tx.candidate_regions(trial, values, capabilities)
    eligible = [m for m in matches if region_contract(m)[1] is None]
    if matches and not eligible:
        reason = region_contract(matches[0])[1]
    return eligible, reason


def export(module, example_inputs, decompose=True, *, capabilities: Iterable[str] = (),
           **export_kwargs):
    """torch.export, optional core-ATen decomposition, then a verified apply."""
    program = torch.export.export(module, tuple(example_inputs), **export_kwargs)
    if decompose:
        program = program.run_decompositions()
    apply(program, verify_with=(module, tuple(example_inputs)), capabilities=capabilities)
    return program


def op_parameters(name: str) -> tuple:
    """Parameters a caller must pass for skeleton `name` (those without a declared default)."""
    skeleton = CG.SKELETONS[name]
    has_default = {symbol for symbol, _ in skeleton.defaults}
    return tuple(arg for symbol, arg in skeleton.params if symbol not in has_default)


def _make_op(name):
    required = op_parameters(name)

    def op(x, *, plan="serial", **params):
        missing = [p for p in required if p not in params]
        if missing:
            raise TypeError(f"neptune_opt.{name}() needs {', '.join(missing)}")
        values = {**CG.param_defaults(name), **params}
        return CG.op_handle(name, params=values or None, plan=plan)(x)

    op.__name__ = op.__qualname__ = name
    op.__doc__ = f"Algebra-derived {name}; explicit serial/split plan on the MI355X HIP backend."
    return op


globals().update({_name: _make_op(_name) for _name in CG.supported()})
__all__ += list(CG.supported())


def optimize(module, example_inputs, *, verbose=False):
    """Deprecated module-returning form of export + apply."""
    warnings.warn("neptune_opt.optimize() is superseded by apply()/export()", DeprecationWarning,
                  stacklevel=2)
    try:
        program = torch.export.export(module, tuple(example_inputs))
    except Exception as error:  # noqa: BLE001
        return module, Report(skipped=[("export-failed", f"{type(error).__name__}: {error}")])
    report = apply(program, verify_with=(module, tuple(example_inputs)))
    if verbose:
        print(report.summary(), file=sys.stderr)
    return (program.module() if report.fusions else module), report


def _rewritten_copy(gm):
    """(graph module to compile, report): a fused trial of gm, or gm itself on any failure."""
    try:
        trial = _tx.fork(gm)
        report = _tx.fuse_regions(trial, None)
    except Exception as error:  # noqa: BLE001
        _raise_if_fatal_cuda(error)
        return gm, Report(skipped=[("rewrite-failed", f"{type(error).__name__}: {error}")])
    return (trial if report.fusions else gm), report


def backend(gm, example_inputs, experimental=False):
    """torch.compile backend (experimental): rewrite, then hand the graph to Inductor."""
    if not experimental:
        raise RuntimeError("neptune_opt.backend is experimental; use export/AOTI, or pass experimental=True")
    import torch._inductor

    global LAST_REPORT
    candidate, LAST_REPORT = _rewritten_copy(gm)
    return torch._inductor.compile(candidate, list(example_inputs))
