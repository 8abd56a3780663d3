"""`compile_best`: ship a fused AOTI package only after it verifies and measurably wins.

Contract of the reference's neptune_opt/ab.py:1-530: the baseline is exported and packaged
untouched; a separately exported candidate goes through `apply` (verified); both packages are
loaded, the candidate must reproduce the baseline's numbers on every supplied case, then the
two are timed in alternating AB/BA rounds and the candidate ships only above `margin` and with
no per-input-key regression beyond `regression_margin`.  Candidate failures fall back to the
baseline; a broken baseline raises; a fatal device-context error always propagates.

On this backend the fused package calls the HIP op through the PyTorch dispatcher (AOTI's
proxy executor), so a process loading the package must have registered the same op -- import
neptune_opt and call the op's handle (e.g. `neptune_codegen.op_handle`) or run `apply` once.
"""
from __future__ import annotations

import contextlib
import copy
import dataclasses
import itertools
import math
import os
import statistics
import tempfile
import time
from collections.abc import Iterable, Sequence

MARGIN = 0.03

# Messages that mean the device context is gone: no in-process fallback is safe after them.
_FATAL_TOKENS = (
    "device-side assert triggered", "cudaerrorassert", "illegal memory access",
    "cudaerrorillegaladdress", "cuda error: unspecified launch failure",
    "cuda context is destroyed", "context is destroyed", "cudaerrorlaunchfailure",
    # HIP spellings
    "hiperrorillegaladdress", "hiperrorlaunchfailure", "hiperrorassert",
    "hip error: unspecified launch failure", "memory access fault", "hiperrorcontextisdestroyed",
    "hiperrorecc", "hiperrornodevice",
)


class FatalCudaError(RuntimeError):
    """The device context is unusable; stop the process rather than fall back in it."""


def _causes(error):
    """error, then everything reachable through __cause__ / __context__, each once."""
    seen, pending = set(), [error]
    while pending:
        current = pending.pop()
        if current is not None and id(current) not in seen:
            seen.add(id(current))
            yield current
            pending += [current.__cause__, current.__context__]


def fatal_cause(error):
    """The exception in error's chain that reports a lost device context, or None."""
    for current in _causes(error):
        if isinstance(current, FatalCudaError):
            return current
        text = str(current).lower()
        if any(token in text for token in _FATAL_TOKENS):
            return current
    return None


def _raise_if_fatal_cuda(error):
    """Raise FatalCudaError when error's chain reports a lost device context; otherwise return.
    Only the message text is inspected: the GPU is not touched."""
    cause = fatal_cause(error)
    if isinstance(cause, FatalCudaError):
        raise cause
    if cause is not None:
        raise FatalCudaError("GPU context failure: stop this process; baseline files may exist "
                             "but in-process execution/fallback is unsafe. Original error: "
                             + str(cause)) from error


@contextlib.contextmanager
def _fatal_errors_escalate():
    """Let exceptions of the body propagate, as FatalCudaError when the device context is lost."""
    try:
        yield
    except Exception as error:  # noqa: BLE001
        _raise_if_fatal_cuda(error)
        raise


@dataclasses.dataclass
class Choice:
    """Which package to ship and the measurements behind the decision."""

    package_path: str
    used_fusion: bool
    baseline_ms: float
    fused_ms: float
    speedup: float
    reason: str
    report: object
    baseline_package: str
    fused_package: str | None = None
    sample_metrics: list[dict] | None = None
    selected_plan: str | None = None
    candidate_metrics: list[dict] | None = None

    def __str__(self) -> str:
        if not math.isfinite(self.baseline_ms) or not math.isfinite(self.fused_ms):
            return f"neptune_opt: {self.reason}"
        which = "fused" if self.used_fusion else "baseline"
        return (f"neptune_opt: shipped the {which} package -- {self.reason} "
                f"(baseline {self.baseline_ms:.4f} ms, fused {self.fused_ms:.4f} ms, "
                f"{self.speedup:.2f}x)")


def _validate_nonnegative(name, value):
    if not math.isfinite(value) or value < 0:
        raise ValueError(f"{name} must be finite and nonnegative")


def choose_faster(baseline_ms: float, fused_ms: float, margin: float = MARGIN) -> tuple:
    """(use fusion, speedup, reason): fusion only for finite positive times and a win > margin."""
    _validate_nonnegative("margin", margin)
    if not all(math.isfinite(t) and t > 0 for t in (baseline_ms, fused_ms)):
        return False, float("nan"), "one of the two packages could not be timed: keeping the baseline"
    speedup = baseline_ms / fused_ms
    if not math.isfinite(speedup) or speedup <= 0:
        return False, float("nan"), "unreliable timing ratio: keeping the baseline"
    if speedup > 1.0 + margin:
        return True, speedup, f"the fused package is {speedup:.2f}x faster"
    if speedup <= 1.0 - margin:
        return False, speedup, f"the fused package is {1 / speedup:.2f}x SLOWER, so it was dropped"
    return False, speedup, (f"the two are within the {margin:.0%} margin ({speedup:.2f}x), so the "
                            "unmodified baseline was kept")


def _name_messages(what, allowed):
    names = "/".join(allowed)
    return {"not_iterable": f"{what} must be a finite iterable of {names} names",
            "string": f"{what} must be a finite iterable of {names} names",
            "bad_item": f"{what} must contain distinct {names} names",
            "too_many": f"{what} must contain at most {len(allowed)} distinct names"}


def _bounded_names(items, allowed, messages):
    """The distinct names of `items`, each one of `allowed`, as a tuple.  At most
    len(allowed) + 1 items are read, so an endless iterable is refused, not exhausted.
    `messages` maps not_iterable / string / bad_item / too_many to the ValueError texts."""
    if isinstance(items, (str, bytes)):
        raise ValueError(messages["string"])
    try:
        iterator = iter(items)
    except TypeError as error:
        raise ValueError(messages["not_iterable"]) from error
    names = []
    for name in itertools.islice(iterator, len(allowed) + 1):
        if not isinstance(name, str) or name not in allowed or name in names:
            raise ValueError(messages["bad_item"])
        names.append(name)
    if len(names) > len(allowed):
        raise ValueError(messages["too_many"])
    return tuple(names)


# ---------------------------------------------------------------- steps (injectable for tests)
def _storage_shared(base, other) -> bool:
    """True when the two programs share their graph module or any state tensor's storage."""
    import torch

    if other is base or other.graph_module is base.graph_module:
        return True
    for name, tensor in base.state_dict.items():
        twin = other.state_dict[name]
        if twin is tensor:
            return True
        if isinstance(tensor, torch.Tensor) and tensor.numel() and tensor.data_ptr() == twin.data_ptr():
            return True
    return False


def _independent_copy(ep_base, module, args, export_kwargs):
    """A program equal to ep_base that shares no graph and no weights with it: a deep copy,
    or, where this torch cannot deep-copy an ExportedProgram faithfully, a fresh export of a
    deep copy of the module (an export of `module` itself would share its parameters)."""
    import torch

    try:
        copied = copy.deepcopy(ep_base)
        if not _storage_shared(ep_base, copied):
            return copied
    except Exception as error:  # noqa: BLE001
        _raise_if_fatal_cuda(error)
    return torch.export.export(copy.deepcopy(module), tuple(args), **export_kwargs)


def _export_pair(module, args, export_kwargs, plan=None, *, baseline=None, capabilities=(),
                 verification_inputs=None, rtol=1e-3, atol=1e-4, max_ulps=None):
    """(baseline program, fused candidate or None, apply's report).  The baseline is exported
    untouched (its errors propagate); the candidate is an independent copy rewritten by a
    verified `apply`.  Any candidate failure becomes a report, never an exception."""
    import torch

    import neptune_opt

    with _fatal_errors_escalate():
        ep_base = baseline if baseline is not None else torch.export.export(
            module, tuple(args), **export_kwargs)
    options = {"rtol": rtol, "atol": atol, "max_ulps": max_ulps}
    if plan is not None:
        options["plan"] = plan
    if capabilities:
        options["capabilities"] = capabilities
    if verification_inputs is not None:
        options["verification_inputs"] = verification_inputs
    try:
        candidate = _independent_copy(ep_base, module, args, export_kwargs)
        report = neptune_opt.apply(candidate, verify_with=(module, tuple(args)), **options)
    except Exception as error:  # noqa: BLE001 -- the optional candidate never breaks the baseline
        _raise_if_fatal_cuda(error)
        return ep_base, None, neptune_opt.Report(
            skipped=[("candidate-failed", f"{type(error).__name__}: {error}")])
    return ep_base, candidate, report


def _package(ep, directory: str, name: str) -> str:
    """AOTI-compile ep into <directory>/<name>.pt2.  The fused HIP ops are dispatcher calls
    (AOTI's proxy executor reaches their C++ kernels), so no user-kernel options apply."""
    import torch

    target = os.path.join(directory, name + ".pt2")
    with _fatal_errors_escalate():
        torch._inductor.aoti_compile_and_package(ep, package_path=target)
    return target


def _load(path: str):
    import torch

    return torch._inductor.aoti_load_package(path)


def _package_output_problem(index, x, y, tol):
    """Why package outputs x and y (leaf `index`) disagree, or None: both must be tensors of
    equal metadata, floating values all finite and within tol, others equal."""
    import torch

    from neptune_opt.verification import _value_difference

    if not (isinstance(x, torch.Tensor) and isinstance(y, torch.Tensor)):
        return f"output {index} is not a tensor"
    if (x.shape, x.dtype, x.device) != (y.shape, y.dtype, y.device):
        return f"output {index} shape/dtype/device differs"
    if not (x.is_floating_point() or x.is_complex()):
        return None if torch.equal(x, y) else f"output {index} integer/bool values differ"
    if not bool(torch.isfinite(x).all()) or not bool(torch.isfinite(y).all()):
        return f"output {index} contains nonfinite values"
    return _value_difference(index, x, y, tol)


def _same_numbers(fa, fb, args, *, rtol: float = 1e-3, atol: float = 1e-4,
                  max_ulps: int | None = None) -> tuple:
    """(ok, detail): fa(*args) and fb(*args) give the same pytree of finite tensors, equal
    within (rtol, atol) -- integers exactly, fp16/bf16 optionally within max_ulps ULPs.  Any
    execution error refuses; a lost device context raises."""
    import torch
    from torch.utils._pytree import tree_flatten

    from neptune_opt.verification import Tolerance

    _validate_nonnegative("rtol", rtol)
    _validate_nonnegative("atol", atol)
    if max_ulps is not None and (type(max_ulps) is not int or max_ulps < 0):
        raise ValueError("max_ulps must be a nonnegative integer or None")
    tol = Tolerance(rtol, atol, max_ulps)
    try:
        with torch.no_grad():
            left, left_spec = tree_flatten(fa(*args))
            right, right_spec = tree_flatten(fb(*args))
        if left_spec != right_spec:
            return False, "output pytree structure differs"
        problems = (_package_output_problem(i, x, y, tol) for i, (x, y) in enumerate(zip(left, right)))
        problem = next((p for p in problems if p), None)
    except Exception as error:  # noqa: BLE001 -- any execution or comparison failure refuses
        _raise_if_fatal_cuda(error)
        return False, f"{type(error).__name__}: {error}"
    return (False, problem) if problem else (True, "")


def _ab_time(fa, fb, args, reps: int = 20, rounds: int = 5, warmup: int = 3) -> tuple:
    """Median ms per call of fa and fb over `rounds` alternating AB / BA rounds of `reps` calls."""
    import torch
    from torch.utils._pytree import tree_flatten

    for name, value, least in (("reps", reps, 1), ("rounds", rounds, 1), ("warmup", warmup, 0)):
        if isinstance(value, bool) or not isinstance(value, int) or value < least:
            raise ValueError(f"{name} must be an integer >= {least}")
    devices = {x.device for x in tree_flatten(args)[0]
               if isinstance(x, torch.Tensor) and x.device.type == "cuda"}

    def sync():
        for device in devices:
            torch.cuda.synchronize(device)

    funcs = (fa, fb)
    samples = ([], [])
    with torch.no_grad():
        for _ in range(warmup):
            fa(*args)
            fb(*args)
        sync()
        for r in range(rounds):
            for side in ((0, 1) if r % 2 == 0 else (1, 0)):
                sync()
                t0 = time.perf_counter()
                for _ in range(reps):
                    funcs[side](*args)
                sync()
                samples[side].append((time.perf_counter() - t0) * 1e3 / reps)
    return statistics.median(samples[0]), statistics.median(samples[1])


def _input_key(args):
    """Structure / shape / stride / dtype / device of the inputs (no tensor data)."""
    import torch
    from torch.utils._pytree import tree_flatten

    leaves, spec = tree_flatten(args)
    return (repr(spec), tuple(
        ("tensor", tuple(x.shape), tuple(x.stride()), str(x.dtype), str(x.device))
        if isinstance(x, torch.Tensor) else (type(x).__qualname__, repr(x)) for x in leaves))


# ---------------------------------------------------------------- the entry point
class _Session:
    """State of one compile_best call: packages, per-case metrics and the decision text."""

    def __init__(self, module, cases, directory, margin, regression_margin, capabilities,
                 verify, tolerances, reps, rounds):
        self.module, self.cases, self.directory = module, cases, directory
        self.margin, self.regression_margin = margin, regression_margin
        self.capabilities, self.verify, self.tolerances = capabilities, verify, tolerances
        self.reps, self.rounds = reps, rounds
        self.scope = f"coverage: {len(cases)} supplied case(s) only, not all dynamic inputs"
        if capabilities:
            self.scope += f"; capabilities: {', '.join(capabilities)}"
        self.base_path = None
        self.baseline = None

    def fresh_metrics(self):
        return [{"case_index": i, "input_key": _input_key(case), "verified": None,
                 "baseline_ms": None, "fused_ms": None, "reason": "not evaluated"}
                for i, case in enumerate(self.cases)]

    def same(self, fa, fb, case):
        return _same_numbers(fa, fb, case, **self.tolerances)

    def choice(self, reason, report, metrics, *, fused_path=None, plan=None, base_ms=float("nan"),
               fused_ms=float("nan"), speedup=1.0, use=False, candidates=None):
        return Choice(fused_path if use else self.base_path, use, base_ms, fused_ms, speedup,
                      f"{reason}; {self.scope}", report, self.base_path, fused_path, metrics,
                      plan if use else None, candidates)

    def evaluate(self, candidate, report, plan, name, candidates):
        """Package, verify and time one candidate; returns its Choice."""
        metrics = self.fresh_metrics()
        if report is None or not report.fusions or candidate is None:
            summary = report.summary().strip() if report is not None else "no candidate report"
            return self.choice(f"nothing to fuse ({summary or 'no fusion'}), so no A/B was run "
                               "for this candidate", report, metrics, candidates=candidates), metrics
        if self.verify and getattr(report, "verified", False) is not True:
            return self.choice("apply report is unverified: the fusion was dropped before "
                               "compilation", report, metrics, candidates=candidates), metrics
        try:
            fused_path = _package(candidate, self.directory, name)
        except Exception as error:  # noqa: BLE001
            _raise_if_fatal_cuda(error)
            return self.choice(f"the fused package failed to compile ({type(error).__name__}: "
                               f"{error}), so the baseline was kept", report, metrics,
                               candidates=candidates), metrics

        def keep(reason):
            return self.choice(reason, report, metrics, fused_path=fused_path, candidates=candidates)

        try:
            fused = _load(fused_path)
            if self.verify:
                failures = []
                for case, metric in zip(self.cases, metrics):
                    ok, detail = self.same(self.baseline, fused, case)
                    metric["verified"], metric["reason"] = ok, detail or "verified"
                    if not ok:
                        failures.append(f"case {metric['case_index']}: {detail}")
                if failures:
                    return keep("the fused package does not reproduce the baseline's numbers "
                                f"({'; '.join(failures)}), so it was dropped"), metrics
            for case, metric in zip(self.cases, metrics):
                base_ms, fused_ms = _ab_time(self.baseline, fused, case, reps=self.reps,
                                             rounds=self.rounds)
                metric.update(baseline_ms=base_ms, fused_ms=fused_ms,
                              reason=choose_faster(base_ms, fused_ms, self.margin)[2])
        except Exception as error:  # noqa: BLE001
            _raise_if_fatal_cuda(error)
            return keep(f"candidate loading/verification/timing failed ({type(error).__name__}: "
                        f"{error}), so the baseline was kept"), metrics
        if any(not all(math.isfinite(m[k]) and m[k] > 0 for k in ("baseline_ms", "fused_ms"))
               for m in metrics):
            return keep("unreliable nonfinite or nonpositive case timing: keeping the baseline"), metrics
        if "segment_pool" in self.capabilities:
            for m in metrics:
                if m["fused_ms"] / m["baseline_ms"] > 1.0 + self.regression_margin:
                    m["reason"] = (f"critical per-case regression (case {m['case_index']}): the "
                                   "fusion is SLOWER on this supplied sample, so it was dropped")
                    return self.choice(m["reason"], report, metrics, fused_path=fused_path,
                                       base_ms=m["baseline_ms"], fused_ms=m["fused_ms"],
                                       speedup=m["baseline_ms"] / m["fused_ms"],
                                       candidates=candidates), metrics
        base_ms = statistics.mean(m["baseline_ms"] for m in metrics)
        fused_ms = statistics.mean(m["fused_ms"] for m in metrics)
        use, speedup, why = choose_faster(base_ms, fused_ms, self.margin)
        by_key: dict = {}
        for m in metrics:
            by_key.setdefault(m["input_key"], []).append(m)
        for group in by_key.values():
            ratio = (statistics.mean(m["fused_ms"] for m in group)
                     / statistics.mean(m["baseline_ms"] for m in group))
            if ratio > 1.0 + self.regression_margin:
                use = False
                why = (f"critical per-key regression (case {group[0]['case_index']}): the fusion "
                       "is SLOWER on this input key, so it was dropped")
                break
        return self.choice(why, report, metrics, fused_path=fused_path, plan=plan, base_ms=base_ms,
                           fused_ms=fused_ms, speedup=speedup, use=use,
                           candidates=candidates), metrics


def compile_best(module, args, *, package_dir: str | None = None, margin: float = MARGIN,
                 reps: int = 20, rounds: int = 5, verify: bool = True,
                 verbose: bool = True, verification_inputs: Sequence[tuple] | None = None,
                 rtol: float = 1e-3, atol: float = 1e-4,
                 regression_margin: float = MARGIN, plans: Iterable[str] = ("serial",),
                 capabilities: Iterable[str] = (), max_ulps: int | None = None,
                 **export_kwargs) -> Choice:
    """Package the unmodified baseline and a fused candidate per plan, verify and A/B time them
    on `args` (+ `verification_inputs`), and return the Choice of what to ship.

    Coverage is the supplied cases only.  `verify=False` skips the correctness checks (an
    explicit opt-out).  `plans` lists candidate plans ("serial", "split"); the fastest eligible
    candidate wins.  `capabilities` enables structured rms_norm / segment_pool fusion; with
    segment_pool every case must avoid a regression above `regression_margin`."""
    import torch

    capabilities = _bounded_names(capabilities, ("rms_norm", "segment_pool"),
                                  _name_messages("capabilities", ("rms_norm", "segment_pool")))
    if max_ulps is not None and (type(max_ulps) is not int or max_ulps < 0):
        raise ValueError("max_ulps must be a nonnegative integer or None")
    for name, value in (("margin", margin), ("regression_margin", regression_margin),
                        ("rtol", rtol), ("atol", atol)):
        _validate_nonnegative(name, value)
    for name, value in (("reps", reps), ("rounds", rounds)):
        if isinstance(value, bool) or not isinstance(value, int) or value < 1:
            raise ValueError(f"{name} must be a positive integer")
    plans = _bounded_names(plans, ("serial", "split"), _name_messages("plans", ("serial", "split")))
    if not plans:
        raise ValueError("plans must not be empty")
    args = tuple(args)
    cases = [args]
    if verification_inputs is not None:
        if not isinstance(verification_inputs, Sequence):
            raise TypeError("verification_inputs must be a sequence of argument tuples")
        if any(not isinstance(case, tuple) for case in verification_inputs):
            raise TypeError("each verification_inputs sample must be an argument tuple")
        cases.extend(verification_inputs)
    if not torch.cuda.is_available():
        raise RuntimeError("compile_best needs a ROCm GPU: it times AOTI packages to decide between "
                           "them. On a CPU-only machine use neptune_opt.export(..., decompose=True).")
    directory = package_dir or tempfile.mkdtemp(prefix="neptune_ab_")
    os.makedirs(directory, exist_ok=True)
    tolerances = {"rtol": rtol, "atol": atol, "max_ulps": max_ulps}
    session = _Session(module, cases, directory, margin, regression_margin, capabilities, verify,
                       tolerances, reps, rounds)
    candidate_kwargs = {"capabilities": capabilities, "verification_inputs": verification_inputs,
                        "rtol": rtol, "atol": atol, "max_ulps": max_ulps}
    ep_base, first_fused, first_report = _export_pair(module, args, export_kwargs, plans[0],
                                                      **candidate_kwargs)
    session.base_path = _package(ep_base, directory, "baseline")   # a broken baseline raises

    def done(choice):
        if verbose:
            print(choice)
        return choice

    try:
        session.baseline = _load(session.base_path)
        if verify:
            failures = []
            for i, case in enumerate(cases):
                ok, detail = session.same(module, session.baseline, case)
                if not ok:
                    failures.append(f"case {i}: {detail}")
            if failures:
                return done(session.choice(
                    f"baseline package numbers verification failed ({'; '.join(failures)}), "
                    "keeping the baseline without a fusion claim", first_report, session.fresh_metrics()))
    except Exception as error:  # noqa: BLE001
        _raise_if_fatal_cuda(error)
        return done(session.choice(f"baseline loading/verification failed ({type(error).__name__}: "
                                   f"{error}), keeping baseline", first_report, session.fresh_metrics()))
    candidates, results = [], []
    for index, plan in enumerate(plans):
        if index == 0:
            ep_fused, report = first_fused, first_report
        else:
            _, ep_fused, report = _export_pair(module, args, export_kwargs, plan, baseline=ep_base,
                                               **candidate_kwargs)
        name = "fused" if plans == ("serial",) else f"fused_{plan}"
        result, metrics = session.evaluate(ep_fused, report, plan, name, candidates)
        candidates.append({"plan": plan, "package_path": result.fused_package,
                           "eligible": result.used_fusion, "selected": False,
                           "baseline_ms": result.baseline_ms, "fused_ms": result.fused_ms,
                           "speedup": result.speedup, "reason": result.reason, "report": report,
                           "sample_metrics": metrics})
        results.append(result)
    eligible = [r for r in results if r.used_fusion]
    if eligible:
        choice = min(eligible, key=lambda r: r.fused_ms)
        for result, entry in zip(results, candidates):
            entry["selected"] = result is choice
        if plans != ("serial",):
            choice.reason = f"selected {choice.selected_plan}: {choice.reason}"
    else:
        choice = results[0]
        if plans != ("serial",):
            choice.reason = "no eligible plan; keeping baseline: " + "; ".join(
                f"{c['plan']}: {c['reason']}" for c in candidates)
    return done(choice)
