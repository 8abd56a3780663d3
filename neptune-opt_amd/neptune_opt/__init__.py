"""neptune_opt -- transactional reduction fusion into MI355X HIP folds.

The public API of the reference package (neptune_opt/__init__.py:26-604): `apply` rewrites
recognised regions of an ExportedProgram into fused HIP ops, verifies them against the
original module on supplied inputs, and publishes the new graph only when every step
succeeded; `preview` reports what `apply` would do; `export` is export + apply; one function
per supported skeleton calls the fused op directly; `compile_best` measures AOTI packages.
Real-algebra matching is a legality check, not an IEEE proof; verification covers the
supplied cases.  A failed trial never changes the caller's graph, signature or weights.
"""
from __future__ import annotations

import copy
import dataclasses
import inspect
import math
import sys
import warnings
from collections.abc import Iterable, Sequence

import torch

import neptune_codegen as CG
from neptune_opt.ab import (Choice, FatalCudaError, _raise_if_fatal_cuda, choose_faster,
                            compile_best)
from neptune_recognize import recognize_regions as _recognize_regions
from neptune_recognize.rewrite import region_contract, rewrite_match

__all__ = ["apply", "export", "optimize", "backend", "preview", "Report", "Fusion",
           "LAST_REPORT", "op_parameters", "compile_best", "Choice"]


@dataclasses.dataclass
class Fusion:
    """One rewritten region."""

    skeleton: str
    params: dict
    input_name: str = ""
    output_name: str = ""
    plan: str = "serial"
    proof_kind: str = ""
    domain_assumptions: tuple = ()
    input_names: tuple = ()
    kind: str = "scalar"
    operation: str = ""
    numeric_contract: tuple = ()

    def __str__(self) -> str:
        if not self.params:
            return self.skeleton
        shown = []
        for key, value in sorted(self.params.items()):
            shown.append(f"{key}={value!r}" if value is None or isinstance(value, bool)
                         else f"{key}={value:g}")
        return f"{self.skeleton}({', '.join(shown)})"


@dataclasses.dataclass
class Report:
    """What apply did: fused regions, refusals, and whether outputs were verified."""

    fusions: list = dataclasses.field(default_factory=list)
    skipped: list = dataclasses.field(default_factory=list)
    verified: bool = False
    graph_changed: bool = False
    verification_cases: int = 0

    def __bool__(self) -> bool:
        return bool(self.fusions)

    def summary(self) -> str:
        lines = [f"  fused   : {fusion}" for fusion in self.fusions]
        lines += [f"  skipped : {reason}: {detail}" for reason, detail in self.skipped]
        if self.fusions:
            lines.append("  verified: fused output matches the supplied inputs" if self.verified
                         else "  unverified: real-algebra match; numerical verification not executed")
        if self.verified and any(f.kind == "structured" for f in self.fusions):
            lines.append("  scope   : supplied-case values and read-only inputs/state; output aliasing not proved")
        return "\n".join(lines) or "  (nothing to do)"


LAST_REPORT: Report | None = None


# ---------------------------------------------------------------- numerical verification
def _clone_inputs(args):
    from torch.utils._pytree import tree_map

    return tree_map(lambda v: v.clone(memory_format=torch.preserve_format)
                    if isinstance(v, torch.Tensor) else v, args)


def _ordered_16bit(value):
    """Monotone integer key of fp16/bf16 bit patterns (+0 and -0 share a key)."""
    bits = value.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    magnitude = bits & 0x7FFF
    return torch.where((bits & 0x8000) != 0, 0x8000 - magnitude, 0x8000 + magnitude)


def _compare_trees(a, b, *, rtol=1e-3, atol=1e-4, max_ulps=None):
    """(equal, detail): same pytree, shapes, dtypes, devices, nonfinite classes and values
    within tolerance (optionally within max_ulps for fp16/bf16)."""
    from torch.utils._pytree import tree_flatten

    left, left_spec = tree_flatten(a)
    right, right_spec = tree_flatten(b)
    if left_spec != right_spec:
        return False, "output pytree structure differs"
    for i, (x, y) in enumerate(zip(left, right)):
        if not isinstance(x, torch.Tensor) or not isinstance(y, torch.Tensor):
            if type(x) is not type(y) or x != y:
                return False, f"non-tensor output {i} differs"
            continue
        if x.shape != y.shape or x.dtype != y.dtype or x.device != y.device:
            return False, f"output {i} shape/dtype/device differs"
        if not (x.is_floating_point() or x.is_complex()):
            if not torch.equal(x, y):
                return False, f"output {i} integer/bool values differ"
            continue
        if not torch.equal(torch.isfinite(x), torch.isfinite(y)):
            return False, f"output {i} finite classification differs"
        if not torch.equal(torch.isnan(x), torch.isnan(y)):
            return False, f"output {i} NaN classification differs"
        if not x.is_complex() and (not torch.equal(torch.isposinf(x), torch.isposinf(y))
                                   or not torch.equal(torch.isneginf(x), torch.isneginf(y))):
            return False, f"output {i} infinity sign differs"
        try:
            torch.testing.assert_close(x, y, rtol=rtol, atol=atol, equal_nan=True)
        except AssertionError as error:
            _raise_if_fatal_cuda(error)
            if max_ulps is None or x.dtype not in (torch.float16, torch.bfloat16):
                return False, f"output {i}: {error}"
            finite = torch.isfinite(x) & torch.isfinite(y)
            distance = (_ordered_16bit(x) - _ordered_16bit(y)).abs()
            if not (distance[finite] <= max_ulps).all():
                return False, f"output {i}: exceeds explicit {max_ulps}-ULP bound"
    return True, ""


def _state_version(tensor):
    try:
        return tensor._version
    except RuntimeError:      # inference tensors have no version counter
        return None


def _snapshot_state(tensors):
    unique = {id(t): t for t in tensors if isinstance(t, torch.Tensor)}
    return [(t, _state_version(t), t.detach().clone()) for t in unique.values()]


def _state_mutated(snapshot):
    return any(_state_version(t) != version or not _compare_trees(t, saved, rtol=0, atol=0)[0]
               for t, version, saved in snapshot)


def _restore_state(snapshot):
    with torch.no_grad():
        for t, version, saved in snapshot:
            if _state_version(t) != version or not _compare_trees(t, saved, rtol=0, atol=0)[0]:
                t.copy_(saved)


def _verify(module, candidate, args, *, rtol=1e-3, atol=1e-4, max_ulps=None):
    """Run module and candidate on clones of args; (ok, detail).  Parameters, buffers and
    inputs must come out unchanged; they are restored either way."""
    try:
        state = _snapshot_state([v for mod in (module, candidate)
                                 for v in (*mod.parameters(), *mod.buffers())])
    except Exception as error:  # noqa: BLE001
        _raise_if_fatal_cuda(error)
        raise
    usable = True
    try:
        with torch.no_grad():
            left, right = _clone_inputs(args), _clone_inputs(args)
            pristine = (_clone_inputs(left), _clone_inputs(right))
            a = module(*left)
            if _state_mutated(state):
                return False, "reference mutated parameters or buffers"
            b = candidate(*right)
            if _state_mutated(state):
                return False, "candidate mutated parameters or buffers"
            for before, after in zip(pristine, (left, right)):
                same, detail = _compare_trees(before, after, rtol=0, atol=0)
                if not same:
                    return False, f"inputs mutated: {detail}"
            return _compare_trees(a, b, rtol=rtol, atol=atol, max_ulps=max_ulps)
    except Exception as error:  # noqa: BLE001 -- an ordinary execution error is a refusal
        try:
            _raise_if_fatal_cuda(error)
        except FatalCudaError:
            usable = False
            raise
        return False, f"{type(error).__name__}: {error}"
    finally:
        if usable:
            try:
                _restore_state(state)
            except Exception as error:  # noqa: BLE001
                _raise_if_fatal_cuda(error)
                raise


# ---------------------------------------------------------------- graph transactions
def _trace(module, args):
    from torch.fx.experimental.proxy_tensor import make_fx

    was_training = module.training
    module.eval()
    try:
        with torch.no_grad():
            return make_fx(module)(*args)
    finally:
        module.train(was_training)


def _graph_trial(gm):
    """A GraphModule with a private copy of the graph and the same (shared) tensors."""
    trial = torch.fx.GraphModule(gm, copy.deepcopy(gm.graph))
    trial.meta = copy.copy(gm.meta)
    if "neptune_replaced_roots" in trial.meta:
        trial.meta["neptune_replaced_roots"] = copy.deepcopy(trial.meta["neptune_replaced_roots"])
    return trial


def _normalize_capabilities(capabilities: Iterable[str]) -> tuple:
    """At most two distinct names from {"rms_norm", "segment_pool"} (reads at most three)."""
    if isinstance(capabilities, (str, bytes)):
        raise ValueError("capabilities must be an iterable of distinct capability names")
    try:
        iterator = iter(capabilities)
    except TypeError as error:
        raise ValueError("capabilities must be an iterable of capability names") from error
    names = []
    for _ in range(3):
        try:
            name = next(iterator)
        except StopIteration:
            return tuple(names)
        if type(name) is not str or name not in ("rms_norm", "segment_pool") or name in names:
            raise ValueError("capabilities must contain only distinct rms_norm/segment_pool names")
        names.append(name)
    raise ValueError("at most two capabilities are supported")


def _discover_regions(gm, values, capabilities):
    """Scalar regions, plus structured ones when capabilities ask for them: complete structured
    regions first, then the largest region per root; refused matches follow the eligible."""
    if not capabilities:
        return _recognize_regions(gm, values)
    from neptune_recognize import recognize_structured_regions

    structured, structured_reason = recognize_structured_regions(gm, capabilities=capabilities)
    scalar, scalar_reason = _recognize_regions(gm, values)
    order = {node: i for i, node in enumerate(gm.graph.nodes)}

    def structured_first(m):
        return getattr(m, "kind", "scalar") != "structured"

    ranked = sorted([*structured, *scalar],
                    key=lambda m: (structured_first(m), -len(m.region_nodes), order[m.region_root]))
    chosen = {}
    for m in ranked:
        if region_contract(m)[1] is None:
            chosen.setdefault(m.region_root, m)
    eligible = sorted(chosen.values(), key=lambda m: (structured_first(m), order[m.region_root]))
    refused = [m for m in ranked if region_contract(m)[1] is not None]
    return [*eligible, *refused], structured_reason or scalar_reason


def _fusion_from_match(match, plan):
    inputs = getattr(match, "input_nodes", ()) or (match.input_node,)
    meta = getattr(match, "metadata", {})
    contract = meta.get("numeric_contract", ())
    if not contract and meta.get("numerical_stages"):
        contract = (meta["numerical_stages"],)
    return Fusion(match.skeleton, dict(match.params), match.input_node.name, match.region_root.name,
                  plan, match.proof_kind, match.domain_assumptions, tuple(n.name for n in inputs),
                  getattr(match, "kind", "scalar"), getattr(match, "operation", ""), tuple(contract))


def _lower_one(gm, values, plan, experimental_log_softmax, report) -> bool:
    """Lower the first compound node whose own expansion is an eligible region, and fuse that
    region in the same transaction.  True when a fusion was committed."""
    from neptune_recognize.lowering import _commit, _is_compound, lower_compound

    for node in list(gm.graph.nodes):
        if not _is_compound(node):
            continue
        if "log_softmax" in str(node.target) and not experimental_log_softmax:
            continue
        tentative = _graph_trial(gm)
        if not lower_compound(tentative, nodes=node.name):
            continue
        found, _ = _recognize_regions(tentative, values)
        chosen = next((m for m in found if m.region_root.meta.get("neptune_lowering") == node.name
                       and region_contract(m)[1] is None), None)
        if chosen is None:
            continue
        fusion = _fusion_from_match(chosen, plan)
        call, refusal = rewrite_match(tentative, chosen, plan=plan)
        if call is None:
            raise RuntimeError(refusal)
        # the lowered node's users now read a value inside or after the fused region; record
        # that rename for the exported signature
        renamed = copy.deepcopy(gm.meta.get("neptune_replaced_roots", {}))
        renamed.update(tentative.meta.get("neptune_replaced_roots", {}))
        users = {u.name for u in node.users}
        for new_user in tentative.graph.nodes:
            if new_user.name not in users:
                continue
            old_user = next(n for n in gm.graph.nodes if n.name == new_user.name)
            old_leaves, _ = torch.utils._pytree.tree_flatten((old_user.args, old_user.kwargs))
            new_leaves, _ = torch.utils._pytree.tree_flatten((new_user.args, new_user.kwargs))
            for old_leaf, new_leaf in zip(old_leaves, new_leaves):
                if old_leaf is node and isinstance(new_leaf, torch.fx.Node):
                    renamed[node.name] = new_leaf.name
        _commit(gm, tentative)
        gm.meta["neptune_replaced_roots"] = renamed
        report.fusions.append(fusion)
        return True
    return False


def _rewrite_regions(gm, values, *, plan="serial", max_regions=None, lower=False,
                     experimental_log_softmax=False, capabilities=()):
    """Fuse regions of `gm` (a trial graph) one at a time, rediscovering after each rewrite."""
    report = Report()
    budget = len(list(gm.graph.nodes)) if max_regions is None else max_regions
    for _ in range(budget):
        matches, reason = _discover_regions(gm, values, capabilities)
        eligible = []
        for m in matches:
            _, refusal = region_contract(m)
            if refusal is None:
                eligible.append(m)
            elif not any(detail == refusal for _, detail in report.skipped):
                report.skipped.append(("refused", refusal))
        if not eligible:
            if lower and _lower_one(gm, values, plan, experimental_log_softmax, report):
                continue
            if not report.fusions and not report.skipped:
                report.skipped.append(("no-fusion", reason))
            break
        match = eligible[0]
        fusion = _fusion_from_match(match, plan)
        call, refusal = rewrite_match(gm, match, plan=plan)
        if call is None:
            raise RuntimeError(refusal)
        report.fusions.append(fusion)
    report.graph_changed = bool(report.fusions)
    return report


def _rewrite_graph(gm, values=None, *, plan="serial", max_regions=None):
    """(candidate, report): a rewritten copy, or `gm` itself on any failure."""
    try:
        trial = _graph_trial(gm)
        report = _rewrite_regions(trial, values, plan=plan, max_regions=max_regions)
        return (trial if report.fusions else gm), report
    except Exception as error:  # noqa: BLE001
        _raise_if_fatal_cuda(error)
        return gm, Report(skipped=[("rewrite-failed", f"{type(error).__name__}: {error}")])


def _candidate_program(exported, trial):
    """An ExportedProgram around the rewritten graph, with its signature and module call graph
    renamed through the recorded root replacements; refuses any other signature change."""
    from torch.export.graph_signature import ConstantArgument
    from torch.utils._pytree import tree_flatten

    signature = copy.deepcopy(exported.graph_signature)
    calls = copy.deepcopy(exported.module_call_graph)
    nodes = {n.name: n for n in trial.graph.nodes}
    replaced = copy.deepcopy(trial.meta.get("neptune_replaced_roots", {}))

    def resolve(name):
        seen = set()
        while name not in nodes:
            if name in seen:
                raise RuntimeError("cyclic rewritten root mapping")
            seen.add(name)
            if name not in replaced:
                raise RuntimeError(f"module signature references removed intermediate {name}")
            name = replaced[name]
        return name

    renamed = {name: resolve(name) for name in replaced if name not in nodes}
    output = next(n for n in trial.graph.nodes if n.op == "output")
    leaves, _ = tree_flatten(output.args[0])
    if len(leaves) != len(signature.output_specs):
        raise RuntimeError("rewrite changed exported output arity")
    for i, (spec, leaf) in enumerate(zip(signature.output_specs, leaves)):
        if isinstance(spec.arg, ConstantArgument):
            if isinstance(leaf, torch.fx.Node) or type(leaf) is not type(spec.arg.value) or leaf != spec.arg.value:
                raise RuntimeError("rewrite changed a constant graph output")
        elif hasattr(spec.arg, "name"):
            if not isinstance(leaf, torch.fx.Node):
                raise RuntimeError("rewrite changed a graph output into a constant")
            if spec.arg.name != leaf.name and (spec.arg.name in nodes or renamed.get(spec.arg.name) != leaf.name):
                raise RuntimeError("rewrite changed output without a root replacement")
            signature.output_specs[i] = dataclasses.replace(
                spec, arg=dataclasses.replace(spec.arg, name=leaf.name))
    for spec in signature.input_specs:
        if hasattr(spec.arg, "name") and spec.arg.name not in nodes:
            raise RuntimeError("rewrite removed an exported graph input")
    for entry in calls:
        if entry.signature is None:
            continue
        for field in ("inputs", "outputs"):
            setattr(entry.signature, field, [
                dataclasses.replace(arg, name=resolve(arg.name))
                if hasattr(arg, "name") and not isinstance(arg, ConstantArgument) else arg
                for arg in getattr(entry.signature, field)])
    kwargs = dict(root=trial, graph=trial.graph, graph_signature=signature,
                  state_dict=exported.state_dict,
                  range_constraints=copy.deepcopy(exported.range_constraints),
                  module_call_graph=calls, example_inputs=exported.example_inputs,
                  constants=exported.constants)
    accepted = inspect.signature(torch.export.ExportedProgram).parameters
    if "verifiers" in accepted:
        kwargs["verifiers"] = list(exported.verifiers)
    elif "verifier" in accepted:
        kwargs["verifier"] = exported.verifier
    return torch.export.ExportedProgram(**kwargs)


def _check_apply_arguments(plan, capabilities, max_regions, rtol, atol, max_ulps,
                           verification_inputs):
    from neptune_codegen.template import validate_plan

    validate_plan(plan)
    capabilities = _normalize_capabilities(capabilities)
    if max_regions is not None and (type(max_regions) is not int or max_regions <= 0):
        raise ValueError("max_regions must be a positive integer or None")
    if any(not math.isfinite(t) or t < 0 for t in (rtol, atol)):
        raise ValueError("verification tolerances must be finite and nonnegative")
    if max_ulps is not None and (type(max_ulps) is not int or max_ulps < 0):
        raise ValueError("max_ulps must be a nonnegative integer or None")
    if verification_inputs is not None:
        if not isinstance(verification_inputs, Sequence):
            raise ValueError("verification_inputs must be a sequence of argument tuples")
        if any(not isinstance(case, tuple) for case in verification_inputs):
            raise ValueError("each verification_inputs sample must be an argument tuple")
    return capabilities


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
    report = Report()
    try:
        capabilities = _check_apply_arguments(plan, capabilities, max_regions, rtol, atol,
                                              max_ulps, verification_inputs)
        signature = exported_program.graph_signature
        if signature.buffers_to_mutate or signature.user_inputs_to_mutate:
            raise ValueError("state/input mutation is outside inference reduction fusion")
        trial = _graph_trial(exported_program.graph_module)
        report = _rewrite_regions(trial, values, plan=plan, max_regions=max_regions, lower=lower,
                                  experimental_log_softmax=experimental_log_softmax,
                                  capabilities=capabilities)
        if not report.fusions:
            LAST_REPORT = report
            return report
        candidate = _candidate_program(exported_program, trial)
        if verify_with is not None:
            module, args = verify_with
            cases = [tuple(args)] + [tuple(c) for c in (verification_inputs or ())]
            executable = candidate.module()
            for index, case in enumerate(cases):
                state = _snapshot_state([*exported_program.state_dict.values(),
                                         *exported_program.constants.values()])
                usable = True
                try:
                    ok, detail = _verify(module, executable, case, rtol=rtol, atol=atol,
                                         max_ulps=max_ulps)
                    if _state_mutated(state):
                        ok, detail = False, "verification mutated original exported state"
                except Exception as error:  # noqa: BLE001
                    try:
                        _raise_if_fatal_cuda(error)
                    except FatalCudaError:
                        usable = False
                        raise
                    raise
                finally:
                    if usable:
                        _restore_state(state)
                if not ok:
                    report = Report(skipped=[("verify-failed", f"case {index}: {detail}")],
                                    verification_cases=index + 1)
                    LAST_REPORT = report
                    return report
            report.verified, report.verification_cases = True, len(cases)
        # everything fallible is done: publish by reference
        exported_program._graph_module = candidate.graph_module
        exported_program._graph_signature = candidate.graph_signature
        exported_program._module_call_graph = candidate.module_call_graph
        report.graph_changed = True
    except Exception as error:  # noqa: BLE001 -- an optional optimisation fails closed
        _raise_if_fatal_cuda(error)
        report = Report(skipped=[("rewrite-failed", f"{type(error).__name__}: {error}")])
    LAST_REPORT = report
    return report


def preview(exported_program, values: dict | None = None, *, lower=True,
            experimental_log_softmax=False, capabilities: Iterable[str] = ()):
    """(eligible matches, reason) that apply would rewrite; generates and launches nothing."""
    from neptune_recognize.lowering import _commit, _is_compound, lower_compound

    capabilities = _normalize_capabilities(capabilities)
    trial = _graph_trial(exported_program.graph_module)
    if lower:
        for node in list(trial.graph.nodes):
            if not _is_compound(node):
                continue
            if "log_softmax" in str(node.target) and not experimental_log_softmax:
                continue
            tentative = _graph_trial(trial)
            if not lower_compound(tentative, nodes=node.name):
                continue
            found, _ = _recognize_regions(tentative, values)
            if any(m.region_root.meta.get("neptune_lowering") == node.name
                   and region_contract(m)[1] is None for m in found):
                _commit(trial, tentative)
    matches, reason = _discover_regions(trial, values, capabilities)
    eligible = [m for m in matches if region_contract(m)[1] is None]
    if matches and not eligible:
        reason = region_contract(matches[0])[1]
    return eligible, reason


def export(module, example_inputs, decompose=True, *, capabilities: Iterable[str] = (),
           **export_kwargs):
    """torch.export, optional core-ATen decomposition, then a verified apply."""
    ep = torch.export.export(module, tuple(example_inputs), **export_kwargs)
    if decompose:
        ep = ep.run_decompositions()
    apply(ep, verify_with=(module, tuple(example_inputs)), capabilities=capabilities)
    return ep


def op_parameters(name: str) -> tuple:
    """Parameters a caller must pass for skeleton `name` (those without a declared default)."""
    sk = CG.SKELETONS[name]
    declared = {sym for sym, _ in sk.defaults}
    return tuple(arg for sym, arg in sk.params if sym not in declared)


def _make_op(name):
    def op(x, *, plan="serial", **params):
        missing = [p for p in op_parameters(name) if p not in params]
        if missing:
            raise TypeError(f"neptune_opt.{name}() needs {', '.join(missing)}")
        values = {**CG.param_defaults(name), **params}
        return CG.op_handle(name, params=values or None, plan=plan)(x)

    op.__name__ = op.__qualname__ = name
    op.__doc__ = f"Algebra-derived {name}; explicit serial/split plan on the MI355X HIP backend."
    return op


for _name in CG.supported():
    globals()[_name] = _make_op(_name)
__all__ += list(CG.supported())


def optimize(module, example_inputs, *, verbose=False):
    """Deprecated module-returning form of export + apply."""
    warnings.warn("neptune_opt.optimize() is superseded by apply()/export()", DeprecationWarning,
                  stacklevel=2)
    try:
        ep = torch.export.export(module, tuple(example_inputs))
    except Exception as error:  # noqa: BLE001
        return module, Report(skipped=[("export-failed", f"{type(error).__name__}: {error}")])
    report = apply(ep, verify_with=(module, tuple(example_inputs)))
    if verbose:
        print(report.summary(), file=sys.stderr)
    return (ep.module() if report.fusions else module), report


def backend(gm, example_inputs, experimental=False):
    """torch.compile backend (experimental): rewrite, then hand the graph to Inductor."""
    if not experimental:
        raise RuntimeError("neptune_opt.backend is experimental; use export/AOTI, or pass experimental=True")
    import torch._inductor

    global LAST_REPORT
    candidate, LAST_REPORT = _rewrite_graph(gm)
    return torch._inductor.compile(candidate, list(example_inputs))
